/* Layout probes of the test-only library libulm_probe.so (built beside
 * libulm_fm.so from csrc/probe.hip and csrc/status.hip; the product library
 * does not contain them). Each launches one wave on the given stream and
 * returns a ulm_status; the library's own ulm_last_error(), declared in
 * ulm_fm.h, holds the message of a failed call. They pin the lane layouts the
 * kernels of libulm_fm.so rely on. No counterpart in the reference. */
#ifndef ULM_PROBE_H
#define ULM_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One v_mfma_f32_32x32x16_bf16 on A = a (32x16 row-major) and B = b (16x32
 * row-major), loaded into the operand lanes the kernels use: d (32x32
 * row-major) = A B, read back from the accumulator lanes the kernels assume. */
int ulm_probe_mfma(const uint16_t *a, const uint16_t *b, float *d, void *stream);

/* LDS transpose read: lane L of one wave addresses elements 4L..4L+3 of the
 * 256 16-bit values in src (staged in LDS) with ds_read_b64_tr_b16 and writes
 * the 4 values it receives to dst[4L..4L+3]. */
int ulm_probe_lds_tr(const uint16_t *src, uint16_t *dst, void *stream);

/* Buffer-to-LDS DMA: lane L loads 16 bytes at byte offset offsets[L] of src
 * (n floats; offsets past the end read as zero) with buffer_load_dwordx4
 * ... lds; the 256-float LDS image is copied to dst. */
int ulm_probe_lds_dma(const float *src, int n, const int *offsets, float *dst, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* ULM_PROBE_H */
