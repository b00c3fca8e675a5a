/*
 * The flint engine's C API, declaration-for-declaration the reference's
 * /root/reference/src/capi.h:1-41 (same names, types, argument meaning and
 * error behaviour), so the Rust server's FFI (/root/reference/server/src/ffi.rs:5-28)
 * links unchanged. Single session, not thread-safe: callers serialise on one thread.
 *
 * In this build the library implements the attention hot path; the GGUF weight
 * loader, the q/k/v/o projections and the MoE FFN are outside it, so
 * flint_open reports that the model weights cannot be served and returns NULL
 * (after the same path checks as the reference). The other functions keep the
 * reference's contract on a handle.
 */
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct flint_engine flint_engine;

typedef struct {
    const char *model_path;   /* GGUF path */
    const char *metallib_dir; /* reference: directory of the Metal libraries; unused here */
    double pool_gb;           /* 0 = all weights resident; >0 expert slot pool (GB); <0 = auto */
    int32_t n_ctx;            /* context length (full-attention KV is sized by it) */
} flint_config;

/* NULL on failure, message in err (may be NULL). /root/reference/src/capi.h:19 */
flint_engine *flint_open(const flint_config *cfg, char *err, int32_t err_len);
void flint_close(flint_engine *e);

int32_t flint_n_ctx(const flint_engine *e);
int32_t flint_n_vocab(void);
int32_t flint_pos(const flint_engine *e);

/* Roll back to pos (<= current). SWA rings keep only the last 1024 positions:
 * after a rollback of more than 511 tokens the caller re-prefills from
 * max(0, pos-512). Returns -1 if pos < 0 or pos > current. */
int32_t flint_truncate(flint_engine *e, int32_t pos);

/* Process n tokens from the current position; greedy next token of the last
 * position, -1 on failure. */
int32_t flint_prefill(flint_engine *e, const int32_t *tokens, int32_t n, char *err, int32_t err_len);
/* Process one token; greedy next token, -1 on failure. */
int32_t flint_decode(flint_engine *e, int32_t token, char *err, int32_t err_len);

/* Logits of the last prefill / decode (flint_n_vocab() floats), valid until the next call. */
const float *flint_logits(const flint_engine *e);

#ifdef __cplusplus
}
#endif
