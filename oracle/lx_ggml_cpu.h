/*
 * lx_ggml_cpu.h — fp32 CPU baseline of the reference's ggml DiT graph
 * (TEST / MEASUREMENT INFRASTRUCTURE ONLY; see lx_ggml_cpu.c).  Weights use the
 * oracle's orc_dit struct (torch layouts, host pointers).
 */
#ifndef LX_GGML_CPU_H
#define LX_GGML_CPU_H

#include "lx_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gcpu_ws gcpu_ws;

/* "avx2" or "avx512": the SGEMM build of this library. */
const char* gcpu_isa(void);
int gcpu_threads(void);
void gcpu_set_threads(int n);

/* Every intermediate tensor of the graph for batch B and up to max_T frames. */
gcpu_ws* gcpu_ws_create(int B, int max_T);
void gcpu_ws_destroy(gcpu_ws* w);

/* time_embed_host: out (1024) for one t. */
void gcpu_time_embed(const orc_dit* wt, float t, float* out);
/* DiT.forward as the reference's graph: x, mu, cond (B, 80, T); spks (B, 80);
 * t (B) host scalars; dphi (B, 80, T).  Returns 0, or -1 on a bad shape. */
int gcpu_dit_forward(gcpu_ws* w, const orc_dit* wt, int B, int T, const float* x,
                     const float* mu, const float* cond, const float* spks, const float* t,
                     float* dphi);
/* One CFG Euler step (B = 2 workspace): x (80, T) in place; mu2, cond2
 * (2, 80, T) and spks2 (2, 80) are the batch-2 graph inputs (row 1 zero). */
int gcpu_cfm_step(gcpu_ws* w, const orc_dit* wt, int T, float* x, const float* mu2,
                  const float* cond2, const float* spks2, float t, float dt, float cfg_rate);

#ifdef __cplusplus
}
#endif

#endif
