/*
 * lx_ggml_cpu.c — fp32 CPU baseline: the reference's ggml graph for one CFG
 * Euler step of the Flow DiT estimator, restated node by node.
 *
 * TEST / MEASUREMENT INFRASTRUCTURE ONLY.  This is the "ggml-equivalent CPU
 * restatement (ggml unavailable offline)" that stands in for the reference's
 * CPU backend (LARYNX_BACKEND=cpu, include/larynx/backend.h:30-33), which
 * cannot be built here because ggml is an un-vendored submodule.  bench.py
 * times it beside the GPU step; tests check it against the oracle.  It is never
 * linked into or called by the product library.
 *
 * What is restated, and how:
 *   - The node sequence of build_dit / dit_block / attention
 *     (src/flow/dit.cpp:34-145) and of the helpers they call
 *     (src/flow/ops.cpp:20-104): every ggml node is one pass over its full
 *     output in fp32, written to its own buffer, in the reference's order.
 *     Views (permute, reshape, view) are strided reads inside the consuming
 *     node, as in ggml; ggml_cont, ggml_concat, ggml_pad_ext, im2col and
 *     repeat are copies.  The attention scores KQ [T, T, 16, B] and their
 *     softmax are materialised (dit.cpp:43-44).
 *   - The host side of the CFM loop (src/flow/flow.cpp:240-259): x_in = [x; x],
 *     time_embed_host in fp32 on one thread (src/flow/flow_matching.cpp:10-42),
 *     the graph, then the CFG combine and x update.
 *   - ggml_mul_mat as a blocked fp32 SGEMM (both operands K-contiguous, B
 *     packed into K x NR and MR x K panels, an MR x NR register tile of FMAs), built for
 *     AVX2+FMA and for AVX-512 (the loader picks the one the host supports).
 *   - Every node runs on all OpenMP threads (ggml's CPU backend splits each
 *     node over its thread pool the same way).
 * Rounding follows plain fp32 evaluation; bit agreement with ggml's own
 * kernels is not claimed (ggml is absent).
 */
#include "lx_ggml_cpu.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* SGEMM  C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]  (ggml_mul_mat(B, A))  */
/* ---------------------------------------------------------------------- */

#if defined(__AVX512F__)
#define GC_VW 16 /* floats per vector register */
#define GC_MR 12
#else
#define GC_VW 8
#define GC_MR 6
#endif
#define GC_NV 2                 /* vectors per tile row */
#define GC_NR (GC_VW * GC_NV)   /* tile columns */
#define GC_KC 256               /* K block */
#define GC_MB (GC_MR * 20)      /* rows of A per work item */
#define GC_NB (GC_NR * 4)       /* columns (B rows) per work item */

typedef float vf __attribute__((vector_size(GC_VW * 4)));
typedef float vfu __attribute__((vector_size(GC_VW * 4), aligned(4)));

const char* gcpu_isa(void) {
#if defined(__AVX512F__)
  return "avx512";
#else
  return "avx2";
#endif
}

int gcpu_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void gcpu_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* B rows n0..n0+nb-1, k0..k0+kc-1 -> panels of GC_NR columns: bp[p][k][j] */
static void pack_b(const float* B, long ldb, int n0, int nb, int k0, int kc, float* bp) {
  for (int p = 0; p < nb; p += GC_NR) {
    float* dst = bp + (long)p * kc;
    for (int j = 0; j < GC_NR; ++j) {
      const int n = p + j;
      if (n < nb) {
        const float* src = B + (long)(n0 + n) * ldb + k0;
        for (int k = 0; k < kc; ++k) dst[(long)k * GC_NR + j] = src[k];
      } else {
        for (int k = 0; k < kc; ++k) dst[(long)k * GC_NR + j] = 0.0f;
      }
    }
  }
}

/* A rows m0..m0+mb-1, k0..k0+kc-1 -> panels of GC_MR rows: ap[p][k][i]
 * (rows past mb repeat the last valid row; their results are not stored). */
static void pack_a(const float* A, long lda, int m0, int mb, int k0, int kc, float* ap) {
  for (int p = 0; p < mb; p += GC_MR) {
    float* dst = ap + (long)p * kc;
    for (int i = 0; i < GC_MR; ++i) {
      const int m = p + i < mb ? p + i : mb - 1;
      const float* src = A + (long)(m0 + m) * lda + k0;
      for (int k = 0; k < kc; ++k) dst[(long)k * GC_MR + i] = src[k];
    }
  }
}

/* MR x NR tile: c[i][j] (+)= sum_k ap[k][i] * bp[k][j]. */
static void micro_tile(int kc, const float* ap, int mr, const float* bp, float* c, long ldc,
                       int nr, int accumulate) {
  vf acc[GC_MR][GC_NV];
  for (int i = 0; i < GC_MR; ++i)
    for (int v = 0; v < GC_NV; ++v) acc[i][v] = (vf){0};
  for (int k = 0; k < kc; ++k) {
    const vf b0 = *(const vf*)(bp + (long)k * GC_NR);
    const vf b1 = *(const vf*)(bp + (long)k * GC_NR + GC_VW);
    const float* a = ap + (long)k * GC_MR;
#pragma GCC unroll 12
    for (int i = 0; i < GC_MR; ++i) {
      const float s = a[i];
      acc[i][0] += s * b0;
      acc[i][1] += s * b1;
    }
  }
  for (int i = 0; i < mr; ++i) {
    float* cr = c + (long)i * ldc;
    if (nr == GC_NR) {
      for (int v = 0; v < GC_NV; ++v) {
        vfu* cp = (vfu*)(cr + v * GC_VW);
        *cp = accumulate ? *cp + acc[i][v] : acc[i][v];
      }
    } else {
      float tmp[GC_NR];
      memcpy(tmp, acc[i], sizeof(tmp));
      for (int j = 0; j < nr; ++j) cr[j] = accumulate ? cr[j] + tmp[j] : tmp[j];
    }
  }
}

/* Batched NT GEMM over nb1 x nb2 batch items with element strides sa*, sb*,
 * sc* per batch dimension.  All threads share the work items (batch, row
 * block, column block), as ggml splits one mul_mat node over its threads. */
static void sgemm_nt(int M, int N, int K, const float* A, long lda, long sa1, long sa2,
                     const float* B, long ldb, long sb1, long sb2, float* C, long ldc, long sc1,
                     long sc2, int nb1, int nb2) {
  const int mblk = (M + GC_MB - 1) / GC_MB;
  const int nblk = (N + GC_NB - 1) / GC_NB;
  const long items = (long)nb1 * nb2 * mblk * nblk;
#pragma omp parallel
  {
    float* bp = (float*)aligned_alloc(64, sizeof(float) * GC_NB * GC_KC);
    float* ap = (float*)aligned_alloc(64, sizeof(float) * (GC_MB + GC_MR) * GC_KC);
#pragma omp for schedule(dynamic, 1)
    for (long it = 0; it < items; ++it) {
      const int mb = (int)(it % mblk);
      const int nbk = (int)((it / mblk) % nblk);
      const long bb = it / ((long)mblk * nblk);
      const int i1 = (int)(bb % nb1), i2 = (int)(bb / nb1);
      const float* Ab = A + i1 * sa1 + i2 * sa2;
      const float* Bb = B + i1 * sb1 + i2 * sb2;
      float* Cb = C + i1 * sc1 + i2 * sc2;
      const int m0 = mb * GC_MB, m1 = m0 + GC_MB < M ? m0 + GC_MB : M;
      const int n0 = nbk * GC_NB, nn = N - n0 < GC_NB ? N - n0 : GC_NB;
      for (int k0 = 0; k0 < K; k0 += GC_KC) {
        const int kc = K - k0 < GC_KC ? K - k0 : GC_KC;
        pack_b(Bb, ldb, n0, nn, k0, kc, bp);
        pack_a(Ab, lda, m0, m1 - m0, k0, kc, ap);
        for (int p = 0; p < nn; p += GC_NR) {
          const int nr = nn - p < GC_NR ? nn - p : GC_NR;
          for (int m = m0; m < m1; m += GC_MR) {
            const int mr = m1 - m < GC_MR ? m1 - m : GC_MR;
            micro_tile(kc, ap + (long)(m - m0) * kc, mr, bp + (long)p * kc,
                       Cb + (long)m * ldc + n0 + p, ldc, nr, k0 > 0);
          }
        }
      }
    }
    free(bp);
    free(ap);
  }
}

/* ---------------------------------------------------------------------- */
/* Elementwise / row nodes (one pass each)                                  */
/* ---------------------------------------------------------------------- */

/* ggml_add(y, b) with b = [N] broadcast over rows: linear's bias node. */
static void node_add_bias(const float* y, const float* b, float* out, long rows, int N) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r)
    for (int i = 0; i < N; ++i) out[r * N + i] = y[r * N + i] + b[i];
}

/* linear(w, b, x) = ggml_add(ggml_mul_mat(w, x), b)  (src/flow/ops.cpp:20-26) */
static void node_linear(const float* x, long ldx, const float* W, const float* bias, float* mm,
                        float* out, int M, int N, int K) {
  sgemm_nt(M, N, K, x, ldx, 0, 0, W, K, 0, 0, mm, N, 0, 0, 1, 1);
  node_add_bias(mm, bias, out, M, N);
}

static void node_silu(const float* x, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = x[i] / (1.0f + expf(-x[i]));
}

/* ggml_norm(x, eps) over rows of D: mean, then the centred mean square. */
static void node_norm(const float* x, float* y, long rows, int D, float eps) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    const float* xr = x + r * D;
    float* yr = y + r * D;
    double s = 0.0;
    for (int i = 0; i < D; ++i) s += xr[i];
    const float mean = (float)(s / D);
    double q = 0.0;
    for (int i = 0; i < D; ++i) {
      const float v = xr[i] - mean;
      yr[i] = v;
      q += (double)v * v;
    }
    const float sc = 1.0f / sqrtf((float)(q / D) + eps);
    for (int i = 0; i < D; ++i) yr[i] *= sc;
  }
}

/* ggml_mul / ggml_add of (B, T, D) with a (B, 1, D) operand. */
static void node_mul_bcast(const float* x, const float* s, float* y, int B, int T, int D) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)B * T; ++r) {
    const float* sr = s + (r / T) * D;
    for (int i = 0; i < D; ++i) y[r * D + i] = x[r * D + i] * sr[i];
  }
}
static void node_add_bcast(const float* x, const float* s, float* y, int B, int T, int D) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)B * T; ++r) {
    const float* sr = s + (r / T) * D;
    for (int i = 0; i < D; ++i) y[r * D + i] = x[r * D + i] + sr[i];
  }
}
static void node_add(const float* a, const float* b, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] + b[i];
}
static void node_mul(const float* a, const float* b, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] * b[i];
}
static void node_scale(const float* a, float s, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] * s;
}
static void node_add_scalar(const float* a, float s, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] + s;
}
static void node_tanh(const float* a, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = tanhf(a[i]);
}
/* ggml_softplus: log(1 + exp(x)), linear above 20 */
static void node_softplus(const float* a, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = a[i] > 20.0f ? a[i] : log1pf(expf(a[i]));
}

/* ada_ln (src/flow/ops.cpp:94-104): norm, add(scale, one), mul, add. */
static void ada_ln(const float* x, const float* scale, const float* shift, float* n, float* s1,
                   float* y, float* out, int B, int T, int D) {
  node_norm(x, n, (long)B * T, D, 1e-6f);
  node_add_scalar(scale, 1.0f, s1, (long)B * D);
  node_mul_bcast(n, s1, y, B, T, D);
  node_add_bcast(y, shift, out, B, T, D);
}

/* gelu_tanh (src/flow/ops.cpp:73-83): nine nodes. */
static void gelu_tanh(const float* x, long n, float* x2, float* x3, float* t0, float* t1,
                      float* out) {
  const float c0 = 0.044715f, c1 = 0.7978845608028654f;
  node_mul(x, x, x2, n);            /* x2 = x * x           */
  node_mul(x2, x, x3, n);           /* x3 = x2 * x          */
  node_scale(x3, c0, t0, n);        /* c0 x^3               */
  node_add(x, t0, t1, n);           /* x + c0 x^3           */
  node_scale(t1, c1, t0, n);        /* * sqrt(2/pi)         */
  node_tanh(t0, t1, n);             /* tanh                 */
  node_add_scalar(t1, 1.0f, t0, n); /* + one                */
  node_scale(x, 0.5f, x2, n);       /* 0.5 x                */
  node_mul(x2, t0, out, n);         /* 0.5 x (1 + tanh)     */
}

/* rope_partial (src/flow/ops.cpp:85-92): ggml_rope_ext NORMAL over the
 * permuted view [D, B, T] (rows of D, position = t), output contiguous in the
 * permuted order, then ggml_cont of the permute back to [D, T, B].  ggml forms
 * theta_i = p * base^(-2i/n_dims) by the recurrence theta *= theta_scale. */
static void rope_partial(const float* q, float* r, float* out, int B, int T, int D, int n_dims,
                         float base) {
  const float theta_scale = powf(base, -2.0f / (float)n_dims);
  /* rope node: r[t][b][:] from q[b][t][:] */
#pragma omp parallel for schedule(static)
  for (long tb = 0; tb < (long)T * B; ++tb) {
    const int t = (int)(tb / B), b = (int)(tb % B);
    const float* src = q + ((long)b * T + t) * D;
    float* dst = r + tb * D;
    float theta = (float)t;
    for (int i = 0; i < n_dims; i += 2) {
      const float c = cosf(theta), s = sinf(theta);
      const float x0 = src[i], x1 = src[i + 1];
      dst[i] = x0 * c - x1 * s;
      dst[i + 1] = x0 * s + x1 * c;
      theta *= theta_scale;
    }
    for (int i = n_dims; i < D; ++i) dst[i] = src[i];
  }
  /* cont(permute): out[b][t][:] = r[t][b][:] */
#pragma omp parallel for schedule(static)
  for (long bt = 0; bt < (long)B * T; ++bt) {
    const int b = (int)(bt / T), t = (int)(bt % T);
    memcpy(out + bt * D, r + ((long)t * B + b) * D, sizeof(float) * D);
  }
}

/* exp(x) for x <= 0 in a form the compiler vectorises (ggml's softmax runs a
 * SIMD exp): Cody-Waite reduction x = n ln2 + r with ln2 split in two parts,
 * e^r by its Taylor series to degree 7 (|r| <= ln2/2, truncation < 6e-9
 * relative), 2^n assembled in the exponent field.  Inputs below -87 flush to
 * e^-87 (below every softmax weight that matters in fp32). */
static inline float exp_nonpos(float x) {
  const float v = x < -87.0f ? -87.0f : x;
  const float n = __builtin_rintf(v * 1.4426950408889634f);
  float r = __builtin_fmaf(n, -0.693145751953125f, v);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  union {
    int32_t i;
    float f;
  } u;
  u.i = ((int32_t)n + 127) << 23;
  return p * u.f;
}

/* ggml_soft_max_ext(KQ, NULL, scale, 0) over rows of n: scaled copy, max,
 * exp and sum, normalise. */
static void node_soft_max(const float* x, float* y, long rows, int n, float scale) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    float* yr = y + r * n;
    float mx = -INFINITY;
#pragma omp simd reduction(max : mx)
    for (int j = 0; j < n; ++j) {
      yr[j] = xr[j] * scale;
      mx = yr[j] > mx ? yr[j] : mx;
    }
    float sum = 0.0f;
#pragma omp simd reduction(+ : sum)
    for (int j = 0; j < n; ++j) {
      yr[j] = exp_nonpos(yr[j] - mx);
      sum += yr[j];
    }
    const float inv = 1.0f / sum;
#pragma omp simd
    for (int j = 0; j < n; ++j) yr[j] *= inv;
  }
}

/* ---------------------------------------------------------------------- */
/* Graph workspace                                                          */
/* ---------------------------------------------------------------------- */

struct gcpu_ws {
  int B, max_T;
  float *cat, *xe_mm, *xe, *pad, *im2col, *cg_mm, *cg, *cg_b, *cat_a, *cat_b, *sp, *th, *c1, *c2,
      *pos_embed, *h, *h2;
  float *silu_t, *emb_mm, *emb, *chunk, *s1, *nrm, *tmp, *xn;
  float *mm, *q, *k, *v, *rq, *rk, *qr, *kr, *kq, *kqs, *vt, *kqv, *att, *att_mm, *y;
  float *f0, *f1, *g0, *g1, *g2, *g3, *g4;
  float *temb, *x_in, *dphi, *proj, *proj_mm;
};

#define WS_FIELDS(X)                                                                        \
  X(cat, BT * 320) X(xe_mm, BT * D) X(xe, BT * D) X(pad, (long)B * (T + 30) * D)             \
  X(im2col, (long)B * T * 64 * 31) X(cg_mm, BT * 64) X(cg, BT * 64) X(cg_b, BT * 64)          \
  X(cat_a, BT * D) X(cat_b, BT * D) X(sp, BT * D) X(th, BT * D) X(c1, BT * D) X(c2, BT * D)   \
  X(pos_embed, BT * D) X(h, BT * D) X(h2, BT * D) X(silu_t, (long)B * D)                     \
  X(emb_mm, (long)B * 6 * D) X(emb, (long)B * 6 * D) X(chunk, (long)6 * B * D)              \
  X(s1, (long)B * D) X(nrm, BT * D) X(tmp, BT * D) X(xn, BT * D) X(mm, BT * 2 * D)          \
  X(q, BT * D) X(k, BT * D) X(v, BT * D) X(rq, BT * D) X(rk, BT * D) X(qr, BT * D)          \
  X(kr, BT * D) X(kq, (long)B * 16 * T * T) X(kqs, (long)B * 16 * T * T) X(vt, BT * D)      \
  X(kqv, BT * D) X(att, BT * D) X(att_mm, BT * D) X(y, BT * D) X(f0, BT * 2 * D)            \
  X(f1, BT * 2 * D) X(g0, BT * 2 * D) X(g1, BT * 2 * D) X(g2, BT * 2 * D) X(g3, BT * 2 * D) \
  X(g4, BT * 2 * D) X(temb, (long)B * D) X(x_in, (long)B * 80 * T) X(dphi, (long)B * 80 * T) \
  X(proj, BT * 80) X(proj_mm, BT * 80)

gcpu_ws* gcpu_ws_create(int B, int max_T) {
  if (B < 1 || max_T < 1) return NULL;
  gcpu_ws* w = (gcpu_ws*)calloc(1, sizeof(gcpu_ws));
  if (!w) return NULL;
  w->B = B;
  w->max_T = max_T;
  const long T = max_T, D = 1024, BT = (long)B * T;
  int ok = 1;
#define WS_ALLOC(name, n)                                                               \
  w->name = (float*)aligned_alloc(64, (((size_t)(n) * sizeof(float)) + 63) / 64 * 64); \
  ok = ok && w->name;
  WS_FIELDS(WS_ALLOC)
#undef WS_ALLOC
  if (!ok) {
    gcpu_ws_destroy(w);
    return NULL;
  }
  return w;
}

void gcpu_ws_destroy(gcpu_ws* w) {
  if (!w) return;
#define WS_FREE(name, n) free(w->name);
  WS_FIELDS(WS_FREE)
#undef WS_FREE
  free(w);
}

/* time_embed_host (src/flow/flow_matching.cpp:10-42): fp32, one thread. */
void gcpu_time_embed(const orc_dit* wt, float t, float* out) {
  float emb[256], h[1024];
  const float log10000_127 = (float)(log(10000.0) / 127.0);
  for (int j = 0; j < 128; ++j) {
    const float coeff = expf(-(float)j * log10000_127);
    const float ang = 1000.0f * t * coeff;
    emb[j] = sinf(ang);
    emb[j + 128] = cosf(ang);
  }
  for (int o = 0; o < 1024; ++o) {
    float acc = wt->time_mlp_0_b[o];
    for (int i = 0; i < 256; ++i) acc += wt->time_mlp_0_w[o * 256 + i] * emb[i];
    h[o] = acc;
  }
  for (int o = 0; o < 1024; ++o) h[o] = h[o] / (1.0f + expf(-h[o]));
  for (int o = 0; o < 1024; ++o) {
    float acc = wt->time_mlp_2_b[o];
    for (int i = 0; i < 1024; ++i) acc += wt->time_mlp_2_w[(long)o * 1024 + i] * h[i];
    out[o] = acc;
  }
}

/* grouped_conv1d (src/flow/ops.cpp:28-67) over the padded input pad [B][C][Tp]
 * (ggml [Tp, C, B]) followed by mish (ops.cpp:69-71); out [B][C][T]. */
static void grouped_conv_mish(gcpu_ws* w, const float* pad, const float* wk, const float* bias,
                              float* out, int B, int T) {
  const int C = 1024, G = 16, cg = 64, K = 31, Tp = T + K - 1;
  const long BT = (long)B * T;
  float* acc_prev = w->cat_a;
  float* acc_next = w->cat_b;
  for (int g = 0; g < G; ++g) {
    /* im2col node: col[b][t][ic*K + kk] = pad[b][g*cg + ic][t + kk] */
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt) {
      const int b = (int)(bt / T), t = (int)(bt % T);
      float* dst = w->im2col + bt * cg * K;
      for (int ic = 0; ic < cg; ++ic) {
        const float* src = pad + ((long)b * C + g * cg + ic) * Tp + t;
        for (int kk = 0; kk < K; ++kk) dst[ic * K + kk] = src[kk];
      }
    }
    /* mul_mat node: cg_mm[oc][bt] = sum_j wk[g*cg + oc][j] * col[bt][j] */
    sgemm_nt(cg, (int)BT, cg * K, wk + (long)g * cg * cg * K, cg * K, 0, 0, w->im2col, cg * K,
             0, 0, w->cg_mm, BT, 0, 0, 1, 1);
    /* reshape [T, B, OC] -> permute [T, OC, B] -> cont node: cg[b][oc][t] */
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)B * cg; ++r) {
      const int b = (int)(r / cg), oc = (int)(r % cg);
      memcpy(w->cg + r * T, w->cg_mm + (long)oc * BT + (long)b * T, sizeof(float) * T);
    }
    /* bias add node: per channel */
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)B * cg; ++r) {
      const float bv = bias[g * cg + (int)(r % cg)];
      for (int t = 0; t < T; ++t) w->cg_b[r * T + t] = w->cg[r * T + t] + bv;
    }
    /* concat node along channels: next[b] = [prev[b] (g*cg ch); cg_b[b]] */
    if (g == 0) {
      memcpy(acc_next, w->cg_b, sizeof(float) * (size_t)B * cg * T);
    } else {
      const long prev_ch = (long)g * cg;
#pragma omp parallel for schedule(static)
      for (long r = 0; r < (long)B * (prev_ch + cg); ++r) {
        const long b = r / (prev_ch + cg), c = r % (prev_ch + cg);
        const float* src = c < prev_ch ? acc_prev + (b * prev_ch + c) * T
                                       : w->cg_b + (b * cg + (c - prev_ch)) * T;
        memcpy(acc_next + r * T, src, sizeof(float) * T);
      }
    }
    float* sw = acc_prev;
    acc_prev = acc_next;
    acc_next = sw;
  }
  /* mish: softplus, tanh, mul (three nodes) */
  const long n = (long)B * C * T;
  node_softplus(acc_prev, w->sp, n);
  node_tanh(w->sp, w->th, n);
  node_mul(acc_prev, w->th, out, n);
}

/* One DiT.forward through the node graph of build_dit (src/flow/dit.cpp:83-145).
 * x_in, mu, cond (B, 80, T) (ggml [T, 80, B]); spks (B, 80); temb (B, 1024). */
static void dit_graph(gcpu_ws* w, const orc_dit* wt, int B, int T, const float* x_in,
                      const float* mu, const float* cond, const float* spks, const float* temb,
                      float* dphi) {
  const int D = 1024, H = 16, HD = 64, F = 2048, mel = 80;
  const long BT = (long)B * T, N = BT * D;
  /* concat[x, cond, mu, spks] over permuted views + the spks repeat (dit.cpp:99-109):
   * three concat nodes and one repeat; materialised as their final result. */
  {
    float* rep = w->tmp; /* repeat node [80, T, B] */
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt)
      memcpy(rep + bt * mel, spks + (bt / T) * mel, sizeof(float) * mel);
    float* c2 = w->nrm; /* concat(x, cond) [160, T, B] */
    float* c3 = w->xn;  /* concat(., mu) [240, T, B]   */
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt) {
      const long b = bt / T, t = bt % T;
      for (int c = 0; c < mel; ++c) {
        c2[bt * 160 + c] = x_in[(b * mel + c) * T + t];
        c2[bt * 160 + mel + c] = cond[(b * mel + c) * T + t];
      }
    }
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt) {
      const long b = bt / T, t = bt % T;
      memcpy(c3 + bt * 240, c2 + bt * 160, sizeof(float) * 160);
      for (int c = 0; c < mel; ++c) c3[bt * 240 + 160 + c] = mu[(b * mel + c) * T + t];
    }
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt) {
      memcpy(w->cat + bt * 320, c3 + bt * 240, sizeof(float) * 240);
      memcpy(w->cat + bt * 320 + 240, rep + bt * mel, sizeof(float) * mel);
    }
  }
  node_linear(w->cat, 320, wt->input_proj_w, wt->input_proj_b, w->xe_mm, w->xe, (int)BT, D, 320);
  /* pad_ext over permute(xe): pad[b][c][30 + t] = xe[b][t][c] */
  const int Tp = T + 30;
#pragma omp parallel for schedule(static)
  for (long bc = 0; bc < (long)B * D; ++bc) {
    const long b = bc / D, c = bc % D;
    float* dst = w->pad + bc * Tp;
    for (int t = 0; t < 30; ++t) dst[t] = 0.0f;
    for (int t = 0; t < T; ++t) dst[30 + t] = w->xe[(b * T + t) * D + c];
  }
  grouped_conv_mish(w, w->pad, wt->conv_pos_1_w, wt->conv_pos_1_b, w->c1, B, T);
  /* pad_ext of c1 [B][C][T] */
#pragma omp parallel for schedule(static)
  for (long bc = 0; bc < (long)B * D; ++bc) {
    float* dst = w->pad + bc * Tp;
    for (int t = 0; t < 30; ++t) dst[t] = 0.0f;
    memcpy(dst + 30, w->c1 + bc * T, sizeof(float) * T);
  }
  grouped_conv_mish(w, w->pad, wt->conv_pos_2_w, wt->conv_pos_2_b, w->c2, B, T);
  /* cont(permute(c2)) -> [1024, T, B], then the residual add */
#pragma omp parallel for schedule(static)
  for (long bt = 0; bt < BT; ++bt) {
    const long b = bt / T, t = bt % T;
    for (int c = 0; c < D; ++c) w->pos_embed[bt * D + c] = w->c2[(b * D + c) * T + t];
  }
  float* h = w->h;
  float* h2 = w->h2;
  node_add(w->xe, w->pos_embed, h, N);

  node_silu(temb, w->silu_t, (long)B * D);
  for (int bi = 0; bi < wt->depth; ++bi) {
    const orc_dit_block* bw = &wt->blocks[bi];
    /* AdaLayerNormZero linear + six view_chunk conts (dit.cpp:56-62) */
    node_linear(w->silu_t, D, bw->attn_norm_w, bw->attn_norm_b, w->emb_mm, w->emb, B, 6 * D, D);
    float* ch[6];
    for (int c = 0; c < 6; ++c) {
      ch[c] = w->chunk + (long)c * B * D;
      for (int b = 0; b < B; ++b)
        memcpy(ch[c] + (long)b * D, w->emb + (long)b * 6 * D + (long)c * D, sizeof(float) * D);
    }
    ada_ln(h, ch[1], ch[0], w->nrm, w->s1, w->tmp, w->xn, B, T, D);
    node_linear(w->xn, D, bw->to_q_w, bw->to_q_b, w->mm, w->q, (int)BT, D, D);
    rope_partial(w->q, w->rq, w->qr, B, T, D, 64, 10000.0f);
    node_linear(w->xn, D, bw->to_k_w, bw->to_k_b, w->mm, w->k, (int)BT, D, D);
    rope_partial(w->k, w->rk, w->kr, B, T, D, 64, 10000.0f);
    node_linear(w->xn, D, bw->to_v_w, bw->to_v_b, w->mm, w->v, (int)BT, D, D);
    /* attention (dit.cpp:34-51): KQ = mul_mat(K, Q) per (head, b) over the
     * permuted views, soft_max_ext, V = cont(permute(v)), KQV = mul_mat(V, KQ),
     * cont(permute(KQV)). */
    sgemm_nt(T, T, HD, w->qr, D, HD, (long)T * D, w->kr, D, HD, (long)T * D, w->kq, T,
             (long)T * T, (long)H * T * T, H, B);
    node_soft_max(w->kq, w->kqs, (long)B * H * T, T, 1.0f / sqrtf((float)HD));
    /* vt[b][h][d][t] = v[b][t][h*HD + d] */
#pragma omp parallel for schedule(static)
    for (long bhd = 0; bhd < (long)B * H * HD; ++bhd) {
      const long b = bhd / (H * HD), hh = (bhd / HD) % H, d = bhd % HD;
      float* dst = w->vt + bhd * T;
      for (int t = 0; t < T; ++t) dst[t] = w->v[(b * T + t) * D + hh * HD + d];
    }
    /* kqv[b][h][t][d] = sum_j kqs[b][h][t][j] vt[b][h][d][j] */
    sgemm_nt(T, HD, T, w->kqs, T, (long)T * T, (long)H * T * T, w->vt, T, (long)HD * T,
             (long)H * HD * T, w->kqv, HD, (long)T * HD, (long)H * T * HD, H, B);
#pragma omp parallel for schedule(static)
    for (long bt = 0; bt < BT; ++bt) {
      const long b = bt / T, t = bt % T;
      for (int hh = 0; hh < H; ++hh)
        memcpy(w->att + bt * D + hh * HD, w->kqv + ((b * H + hh) * T + t) * HD,
               sizeof(float) * HD);
    }
    node_linear(w->att, D, bw->to_out_w, bw->to_out_b, w->att_mm, w->y, (int)BT, D, D);
    node_mul_bcast(w->y, ch[2], w->tmp, B, T, D);
    node_add(h, w->tmp, h2, N);
    { float* s = h; h = h2; h2 = s; }
    ada_ln(h, ch[4], ch[3], w->nrm, w->s1, w->tmp, w->xn, B, T, D);
    node_linear(w->xn, D, bw->ff0_w, bw->ff0_b, w->mm, w->f0, (int)BT, F, D);
    gelu_tanh(w->f0, BT * F, w->g0, w->g1, w->g2, w->g3, w->f1);
    node_linear(w->f1, F, bw->ff2_w, bw->ff2_b, w->att_mm, w->y, (int)BT, D, F);
    node_mul_bcast(w->y, ch[5], w->tmp, B, T, D);
    node_add(h, w->tmp, h2, N);
    { float* s = h; h = h2; h2 = s; }
  }
  /* norm_out (dit.cpp:133-136): linear, scale / shift conts, ada_ln */
  node_linear(w->silu_t, D, wt->norm_out_w, wt->norm_out_b, w->emb_mm, w->emb, B, 2 * D, D);
  float* scale = w->chunk;
  float* shift = w->chunk + (long)B * D;
  for (int b = 0; b < B; ++b) {
    memcpy(scale + (long)b * D, w->emb + (long)b * 2 * D, sizeof(float) * D);
    memcpy(shift + (long)b * D, w->emb + (long)b * 2 * D + D, sizeof(float) * D);
  }
  ada_ln(h, scale, shift, w->nrm, w->s1, w->tmp, w->xn, B, T, D);
  node_linear(w->xn, D, wt->proj_out_w, wt->proj_out_b, w->proj_mm, w->proj, (int)BT, mel, D);
  /* cont(permute(proj)) -> [T, 80, B] */
#pragma omp parallel for schedule(static)
  for (long bc = 0; bc < (long)B * mel; ++bc) {
    const long b = bc / mel, c = bc % mel;
    for (int t = 0; t < T; ++t) dphi[bc * T + t] = w->proj[(b * T + t) * mel + c];
  }
}

int gcpu_dit_forward(gcpu_ws* w, const orc_dit* wt, int B, int T, const float* x,
                     const float* mu, const float* cond, const float* spks, const float* t,
                     float* dphi) {
  if (!w || B != w->B || T < 1 || T > w->max_T || wt->dim != 1024 || wt->heads != 16 ||
      wt->head_dim != 64 || wt->ff_inner != 2048 || wt->mel_dim != 80)
    return -1;
  for (int b = 0; b < B; ++b) gcpu_time_embed(wt, t[b], w->temb + (long)b * 1024);
  dit_graph(w, wt, B, T, x, mu, cond, spks, w->temb, dphi);
  return 0;
}

/* One CFG Euler step as FlowDecoder::infer runs it (src/flow/flow.cpp:240-259):
 * x (80, T) in place; mu, cond (80, T); spks (80).  The workspace holds the
 * batch-2 inputs, as the reference's graph input tensors do. */
int gcpu_cfm_step(gcpu_ws* w, const orc_dit* wt, int T, float* x, const float* mu2,
                  const float* cond2, const float* spks2, float t, float dt, float cfg_rate) {
  if (!w || w->B != 2 || T < 1 || T > w->max_T) return -1;
  const long n = 80L * T;
  memcpy(w->x_in, x, sizeof(float) * n);
  memcpy(w->x_in + n, x, sizeof(float) * n);
  gcpu_time_embed(wt, t, w->temb);
  memcpy(w->temb + 1024, w->temb, sizeof(float) * 1024);
  dit_graph(w, wt, 2, T, w->x_in, mu2, cond2, spks2, w->temb, w->dphi);
  const float a = 1.0f + cfg_rate, b = cfg_rate;
  for (long i = 0; i < n; ++i) x[i] += dt * (a * w->dphi[i] - b * w->dphi[i + n]);
  return 0;
}
