/*
 * Parity shim around the reference's own C decoder (run.c:193-265).
 *
 * TEST INFRASTRUCTURE ONLY. This file is compiled together with the
 * reference's unmodified run.c, included from where it lies (the Makefile
 * passes its path as RUNC_SOURCE); nothing of run.c is copied here. Its CLI
 * entry point is renamed so the translation unit can be a shared library, and
 * four entry points expose run.c's own read_checkpoint / reset_state /
 * forward so a test can feed tokens one at a time and read back the logits.
 */
#define main runc_reference_cli_main
#include RUNC_SOURCE
#undef main

static UnifiedLM g_ref;
static int g_ref_loaded = 0;

/* Loads a ULMe v1 checkpoint (run.c:140-186) and resets the decode state. */
int runc_ref_load(const char *path) {
    if (g_ref_loaded) {
        free_model(&g_ref);
        memset(&g_ref, 0, sizeof(g_ref));
    }
    read_checkpoint(path, &g_ref);
    malloc_run_state(&g_ref.state, &g_ref.config);
    reset_state(&g_ref);
    g_ref_loaded = 1;
    return 0;
}

/* State back to the prior (run.c:121-138). */
void runc_ref_reset(void) { reset_state(&g_ref); }

/* One position of run.c's forward (run.c:193-265); returns its logits buffer. */
const float *runc_ref_forward(int token) { return forward(&g_ref, token); }

int runc_ref_vocab(void) { return g_ref.config.vocab_size; }
