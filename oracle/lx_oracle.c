/*
 * lx_oracle.c — CPU oracle (test infrastructure; see lx_oracle.h).
 *
 * Each function names the reference lines whose algorithm it restates.  Paths
 * are relative to the Larynx source tree.
 */
#include "lx_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* splitmix64 finaliser (Steele, Lea, Flood 2014). */
static uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* Counter-based N(0, std^2) fill: element pair p draws two 53-bit uniforms
 * from mix64(key + 2p), mix64(key + 2p + 1) and applies Box-Muller.  Any
 * (seed, stream) regenerates the same tensor on any host. */
void orc_fill_normal(float* out, long n, uint64_t seed, uint64_t stream, float std) {
  const uint64_t key = mix64(mix64(seed) ^ (stream * 0xD1B54A32D192ED03ULL));
  const long npair = (n + 1) / 2;
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (long p = 0; p < npair; ++p) {
    const uint64_t z1 = mix64(key + 2 * (uint64_t)p);
    const uint64_t z2 = mix64(key + 2 * (uint64_t)p + 1);
    const double u1 = ((double)(z1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(z2 >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1)) * (double)std;
    out[2 * p] = (float)(r * cos(two_pi * u2));
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(r * sin(two_pi * u2));
  }
}

/* ada_ln: ggml_norm(eps) (biased variance, no affine) * (1 + scale) + shift.
 * src/flow/ops.cpp:94-104; AdaLayerNormZero flow_reference.py:169-180. */
void orc_adaln(const float* x, const float* shift, const float* scale, long mod_stride, float* y,
               int B, int T, int D, float eps) {
  long rows = (long)B * T;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    const float* xr = x + r * D;
    const int b = (int)(r / T);
    double s = 0.0;
    for (int i = 0; i < D; ++i) s += xr[i];
    const double mean = s / D;
    double q = 0.0;
    for (int i = 0; i < D; ++i) {
      double c = xr[i] - mean;
      q += c * c;
    }
    const double rstd = 1.0 / sqrt(q / D + (double)eps);
    const float* sh = shift + (long)b * mod_stride;
    const float* sc = scale + (long)b * mod_stride;
    float* yr = y + r * D;
    for (int i = 0; i < D; ++i)
      yr[i] = (float)(((double)xr[i] - mean) * rstd * (1.0 + (double)sc[i]) + (double)sh[i]);
  }
}

/* linear: y = x W^T + b, W (N, K) = ggml [K, N].  src/flow/ops.cpp:20-26,
 * src/llm/ops.cpp:13-19.  fp64 accumulation, 4x4 register blocks, W tiles of
 * 64 rows kept hot per thread. */
void orc_linear(const float* x, int ldx, const float* W, const float* bias, float* y, int ldy,
                int M, int N, int K) {
  const int NB = 64;
  const int nblk = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1)
  for (int blk = 0; blk < nblk; ++blk) {
    const int n0 = blk * NB, n1 = n0 + NB < N ? n0 + NB : N;
    for (int m = 0; m < M; m += 4) {
      const int mc = M - m < 4 ? M - m : 4;
      for (int n = n0; n < n1; n += 4) {
        const int nc = n1 - n < 4 ? n1 - n : 4;
        double acc[4][4] = {{0}};
        const float* xr[4];
        const float* wr[4];
        for (int i = 0; i < 4; ++i) xr[i] = x + (long)(m + (i < mc ? i : 0)) * ldx;
        for (int j = 0; j < 4; ++j) wr[j] = W + (long)(n + (j < nc ? j : 0)) * K;
        double a00 = 0, a01 = 0, a02 = 0, a03 = 0, a10 = 0, a11 = 0, a12 = 0, a13 = 0;
        double a20 = 0, a21 = 0, a22 = 0, a23 = 0, a30 = 0, a31 = 0, a32 = 0, a33 = 0;
#pragma omp simd reduction(+ : a00, a01, a02, a03, a10, a11, a12, a13, a20, a21, a22, a23, a30, \
                               a31, a32, a33)
        for (int k = 0; k < K; ++k) {
          const double x0 = xr[0][k], x1 = xr[1][k], x2 = xr[2][k], x3 = xr[3][k];
          const double w0 = wr[0][k], w1 = wr[1][k], w2 = wr[2][k], w3 = wr[3][k];
          a00 += x0 * w0; a01 += x0 * w1; a02 += x0 * w2; a03 += x0 * w3;
          a10 += x1 * w0; a11 += x1 * w1; a12 += x1 * w2; a13 += x1 * w3;
          a20 += x2 * w0; a21 += x2 * w1; a22 += x2 * w2; a23 += x2 * w3;
          a30 += x3 * w0; a31 += x3 * w1; a32 += x3 * w2; a33 += x3 * w3;
        }
        acc[0][0] = a00; acc[0][1] = a01; acc[0][2] = a02; acc[0][3] = a03;
        acc[1][0] = a10; acc[1][1] = a11; acc[1][2] = a12; acc[1][3] = a13;
        acc[2][0] = a20; acc[2][1] = a21; acc[2][2] = a22; acc[2][3] = a23;
        acc[3][0] = a30; acc[3][1] = a31; acc[3][2] = a32; acc[3][3] = a33;
        for (int i = 0; i < mc; ++i)
          for (int j = 0; j < nc; ++j)
            y[(long)(m + i) * ldy + n + j] =
                (float)(acc[i][j] + (bias ? (double)bias[n + j] : 0.0));
      }
    }
  }
}

static double silu_d(double v) { return v / (1.0 + exp(-v)); }

void orc_silu_vec(const float* x, float* y, long n) {
  for (long i = 0; i < n; ++i) y[i] = (float)silu_d(x[i]);
}

/* gelu_tanh: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
 * src/flow/ops.cpp:73-83; nn.GELU("tanh") flow_reference.py:282. */
static double gelu_d(double x) {
  const double c0 = 0.044715, c1 = 0.7978845608028654;
  return 0.5 * x * (1.0 + tanh(c1 * (x + c0 * x * x * x)));
}

void orc_gelu_tanh(const float* h, float* y, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) y[i] = (float)gelu_d(h[i]);
}

/* gated residual: x += gate_b * y.  src/flow/dit.cpp:71, 77. */
void orc_gated_residual(float* x, const float* y, const float* gate, long gate_stride, int B,
                        int T, int D) {
  long rows = (long)B * T;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    const float* g = gate + (r / T) * gate_stride;
    for (int i = 0; i < D; ++i)
      x[r * D + i] = (float)((double)x[r * D + i] + (double)g[i] * (double)y[r * D + i]);
  }
}

/* inv_freq = 1 / base^(arange(0, dim, 2) / dim) in fp32: pow rounded to fp32,
 * then an fp32 reciprocal (flow_reference.py:79), which reproduces torch's
 * table bit for bit for base 1e4 and 1e6. */
void orc_rope_inv_freq(float base, int dim, float* out) {
  for (int i = 0; i < dim / 2; ++i) {
    float e = (float)(2 * i) / (float)dim;
    float p = (float)pow((double)base, (double)e);
    out[i] = 1.0f / p;
  }
}

/* rope_partial: GPT-J interleaved pairs (2i, 2i+1) on channels < rot_dim,
 * angle = fp32(pos) * inv_freq[i] (fp32).  src/flow/ops.cpp:85-92;
 * apply_rotary_pos_emb / rotate_half flow_reference.py:52-71. */
void orc_rope_partial(float* q, const int* pos, int B, int T, int ld, int rot_dim, float base) {
  float inv[128];
  orc_rope_inv_freq(base, rot_dim, inv);
  long rows = (long)B * T;
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; ++r) {
    const float p = (float)pos[r % T];
    float* row = q + r * ld;
    for (int i = 0; i < rot_dim / 2; ++i) {
      const float ang = p * inv[i];
      const double c = cos((double)ang), s = sin((double)ang);
      const double x0 = row[2 * i], x1 = row[2 * i + 1];
      row[2 * i] = (float)(x0 * c - x1 * s);
      row[2 * i + 1] = (float)(x1 * c + x0 * s);
    }
  }
}

/* Sinusoid of time_embed_host (src/flow/flow_matching.cpp:14-20):
 * coeff_j = expf(-j * fp32(ln(1e4)/(half-1))), angle = (scale * t) * coeff_j in
 * fp32, then sin / cos. */
void orc_timestep_embed(const float* t, int B, int half_dim, float scale, float* out) {
  const float step = (float)(log(10000.0) / (double)(half_dim - 1));
  for (int b = 0; b < B; ++b) {
    const float ts = scale * t[b];
    for (int j = 0; j < half_dim; ++j) {
      const float coeff = expf(-(float)j * step);
      const float ang = ts * coeff;
      out[(long)b * 2 * half_dim + j] = (float)sin((double)ang);
      out[(long)b * 2 * half_dim + half_dim + j] = (float)cos((double)ang);
    }
  }
}

/* TimestepEmbedding: sinusoid(256, scale 1000) -> Linear -> SiLU -> Linear.
 * src/flow/flow_matching.cpp:10-42; flow_reference.py:294-304. */
void orc_time_mlp(const float* t, int B, const float* w0, const float* b0, const float* w2,
                  const float* b2, int D, float* out) {
  float* sinus = (float*)malloc(sizeof(float) * B * 256);
  float* h = (float*)malloc(sizeof(float) * B * D);
  orc_timestep_embed(t, B, 128, 1000.0f, sinus);
  orc_linear(sinus, 256, w0, b0, h, D, B, D, 256);
  for (long i = 0; i < (long)B * D; ++i) h[i] = (float)silu_d(h[i]);
  orc_linear(h, D, w2, b2, out, D, B, D, D);
  free(sinus);
  free(h);
}

/* rms_norm: x / sqrt(mean(x^2) + eps) * w.  src/llm/ops.cpp:7-11. */
void orc_rmsnorm(const float* x, const float* w, float* y, int rows, int D, float eps) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (long)r * D;
    double s = 0.0;
    for (int i = 0; i < D; ++i) s += (double)xr[i] * xr[i];
    const double rr = 1.0 / sqrt(s / D + (double)eps);
    for (int i = 0; i < D; ++i) y[(long)r * D + i] = (float)((double)xr[i] * rr * (double)w[i]);
  }
}

/* rope_full NEOX: pairs (i, i + hd/2) per head, theta^(-2i/hd).
 * src/llm/ops.cpp:21-30 (GGML_ROPE_TYPE_NEOX, theta 1e6 src/llm/internal.h:28). */
void orc_rope_neox(float* qk, const int* pos, int rows, int n_heads, int head_dim, int ld,
                   float theta) {
  float inv[128];
  orc_rope_inv_freq(theta, head_dim, inv);
  const int half = head_dim / 2;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float p = (float)pos[r];
    for (int h = 0; h < n_heads; ++h) {
      float* v = qk + (long)r * ld + h * head_dim;
      for (int i = 0; i < half; ++i) {
        const float ang = p * inv[i];
        const double c = cos((double)ang), s = sin((double)ang);
        const double x0 = v[i], x1 = v[i + half];
        v[i] = (float)(x0 * c - x1 * s);
        v[i + half] = (float)(x1 * c + x0 * s);
      }
    }
  }
}

/* SwiGLU gate: silu(gate) * up.  src/llm/llm.cpp:167-169. */
void orc_swiglu(const float* gate, const float* up, float* out, long n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = (float)(silu_d(gate[i]) * (double)up[i]);
}

/* Row gather, all ids validated first.  src/llm/llm.cpp:63-100. */
int orc_embed_gather(const float* table, long n_rows, int D, const int* ids, int n, float* out) {
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || (long)ids[i] >= n_rows) return -3;
  for (int i = 0; i < n; ++i)
    memcpy(out + (long)i * D, table + (long)ids[i] * D, sizeof(float) * D);
  return 0;
}

/* softmax(scale q k^T [+ causal]) v per head, GQA head h -> kv h / rep.
 * src/flow/dit.cpp:34-51; src/llm/ops.cpp:32-65.  Scores, softmax and P.V
 * are evaluated in fp64.  Work is blocked for speed only (4 queries against 4
 * keys per register tile, K and V converted to fp64 once): every score is a
 * full fp64 dot product and every output an fp64 sum, whatever the order. */
enum { ORC_QB = 4 };
void orc_attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv,
                   float* o, int ldo, int B, int Tq, int Tk, int n_heads, int n_kv_heads,
                   int head_dim, float scale, int causal, int q_offset) {
  const int rep = n_heads / n_kv_heads;
  const int hd = head_dim;
  const long kv_elems = (long)B * n_kv_heads * Tk * hd;
  double* kd = (double*)malloc(sizeof(double) * (kv_elems > 0 ? kv_elems : 1));
  double* vd = (double*)malloc(sizeof(double) * (kv_elems > 0 ? kv_elems : 1));
  if (!kd || !vd) {
    free(kd);
    free(vd);
    return;
  }
  /* (b, g, j, d) contiguous fp64 copies */
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)B * n_kv_heads * Tk; ++r) {
    const int j = (int)(r % Tk);
    const int g = (int)((r / Tk) % n_kv_heads);
    const int b = (int)(r / ((long)Tk * n_kv_heads));
    const float* kr = k + ((long)b * Tk + j) * ldk + g * hd;
    const float* vr = v + ((long)b * Tk + j) * ldv + g * hd;
    for (int d = 0; d < hd; ++d) {
      kd[r * hd + d] = kr[d];
      vd[r * hd + d] = vr[d];
    }
  }
  const int nqb = (Tq + ORC_QB - 1) / ORC_QB;
  const long work = (long)B * n_heads * nqb;
#pragma omp parallel
  {
    double* sc = (double*)malloc(sizeof(double) * ORC_QB * (Tk > 0 ? Tk : 1));
    double* qv = (double*)malloc(sizeof(double) * ORC_QB * hd);
    double* acc = (double*)malloc(sizeof(double) * ORC_QB * hd);
#pragma omp for schedule(dynamic, 4)
    for (long w = 0; w < work; ++w) {
      const int qb = (int)(w % nqb);
      const int h = (int)((w / nqb) % n_heads);
      const int b = (int)(w / ((long)nqb * n_heads));
      const int g = h / rep;
      const int i0 = qb * ORC_QB;
      const int nq = Tq - i0 < ORC_QB ? Tq - i0 : ORC_QB;
      int kend[ORC_QB];
      int kmax = 0;
      for (int ii = 0; ii < ORC_QB; ++ii) {
        const int i = i0 + (ii < nq ? ii : nq - 1); /* pad rows repeat the last query */
        const float* qr = q + ((long)b * Tq + i) * ldq + h * hd;
        for (int d = 0; d < hd; ++d) qv[ii * hd + d] = qr[d];
        kend[ii] = causal ? (q_offset + i + 1 < Tk ? q_offset + i + 1 : Tk) : Tk;
        if (kend[ii] > kmax) kmax = kend[ii];
      }
      const double* kb = kd + ((long)b * n_kv_heads + g) * Tk * hd;
      const double* vb = vd + ((long)b * n_kv_heads + g) * Tk * hd;
      const double* q0 = qv;
      const double* q1 = qv + hd;
      const double* q2 = qv + 2 * hd;
      const double* q3 = qv + 3 * hd;
      for (int j0 = 0; j0 < kmax; j0 += 4) {
        const int nj = kmax - j0 < 4 ? kmax - j0 : 4;
        const double* k0 = kb + (long)j0 * hd;
        const double* k1 = kb + (long)(j0 + (nj > 1 ? 1 : 0)) * hd;
        const double* k2 = kb + (long)(j0 + (nj > 2 ? 2 : 0)) * hd;
        const double* k3 = kb + (long)(j0 + (nj > 3 ? 3 : 0)) * hd;
        double s00 = 0, s01 = 0, s02 = 0, s03 = 0, s10 = 0, s11 = 0, s12 = 0, s13 = 0;
        double s20 = 0, s21 = 0, s22 = 0, s23 = 0, s30 = 0, s31 = 0, s32 = 0, s33 = 0;
#pragma omp simd reduction(+ : s00, s01, s02, s03, s10, s11, s12, s13, s20, s21, s22, s23, s30, \
                               s31, s32, s33)
        for (int d = 0; d < hd; ++d) {
          s00 += q0[d] * k0[d]; s01 += q0[d] * k1[d]; s02 += q0[d] * k2[d]; s03 += q0[d] * k3[d];
          s10 += q1[d] * k0[d]; s11 += q1[d] * k1[d]; s12 += q1[d] * k2[d]; s13 += q1[d] * k3[d];
          s20 += q2[d] * k0[d]; s21 += q2[d] * k1[d]; s22 += q2[d] * k2[d]; s23 += q2[d] * k3[d];
          s30 += q3[d] * k0[d]; s31 += q3[d] * k1[d]; s32 += q3[d] * k2[d]; s33 += q3[d] * k3[d];
        }
        const double s4[4][4] = {{s00, s01, s02, s03}, {s10, s11, s12, s13},
                                 {s20, s21, s22, s23}, {s30, s31, s32, s33}};
        for (int ii = 0; ii < ORC_QB; ++ii)
          for (int jj = 0; jj < nj; ++jj) sc[(long)ii * Tk + j0 + jj] = s4[ii][jj] * scale;
      }
      double l[ORC_QB];
      for (int ii = 0; ii < ORC_QB; ++ii) {
        double* sr = sc + (long)ii * Tk;
        double mx = -INFINITY;
        for (int j = 0; j < kend[ii]; ++j)
          if (sr[j] > mx) mx = sr[j];
        double sum = 0.0;
        for (int j = 0; j < kend[ii]; ++j) {
          sr[j] = exp(sr[j] - mx);
          sum += sr[j];
        }
        for (int j = kend[ii]; j < kmax; ++j) sr[j] = 0.0;
        l[ii] = sum;
      }
      for (int x = 0; x < ORC_QB * hd; ++x) acc[x] = 0.0;
      for (int j = 0; j < kmax; ++j) {
        const double* vr = vb + (long)j * hd;
        const double p0 = sc[j], p1 = sc[Tk + j], p2 = sc[2L * Tk + j], p3 = sc[3L * Tk + j];
        double* a0 = acc;
        double* a1 = acc + hd;
        double* a2 = acc + 2 * hd;
        double* a3 = acc + 3 * hd;
#pragma omp simd
        for (int d = 0; d < hd; ++d) {
          a0[d] += p0 * vr[d];
          a1[d] += p1 * vr[d];
          a2[d] += p2 * vr[d];
          a3[d] += p3 * vr[d];
        }
      }
      for (int ii = 0; ii < nq; ++ii) {
        float* orow = o + ((long)b * Tq + i0 + ii) * ldo + h * hd;
        for (int d = 0; d < hd; ++d) orow[d] = (float)(acc[ii * hd + d] / l[ii]);
      }
    }
    free(sc);
    free(qv);
    free(acc);
  }
  free(kd);
  free(vd);
}

static double mish_d(double x) {
  /* torch softplus threshold 20 */
  const double sp = x > 20.0 ? x : log1p(exp(x));
  return x * tanh(sp);
}

/* Left-padded grouped conv1d + bias + Mish (+ residual).
 * src/flow/dit.cpp:113-122, src/flow/ops.cpp:28-71;
 * CausalConvPositionEmbedding flow_reference.py:140-166.  w: (C, C/G, K). */
void orc_conv_pos_mish(const float* x, const float* w, const float* bias, const float* resid,
                       float* y, int B, int T, int C, int G, int K) {
  const int cg = C / G;
  const long work = (long)B * T;
#pragma omp parallel for schedule(static)
  for (long bt = 0; bt < work; ++bt) {
    const int b = (int)(bt / T), t = (int)(bt % T);
    for (int oc = 0; oc < C; ++oc) {
      const int g = oc / cg;
      double s = bias ? (double)bias[oc] : 0.0;
      for (int kk = 0; kk < K; ++kk) {
        const int ts = t - (K - 1) + kk;
        if (ts < 0) continue;
        const float* xr = x + ((long)b * T + ts) * C + g * cg;
        const float* wr = w + (long)oc * cg * K + kk;
        for (int ic = 0; ic < cg; ++ic) s += (double)wr[(long)ic * K] * xr[ic];
      }
      double v = mish_d(s);
      if (resid) v += (double)resid[bt * C + oc];
      y[bt * C + oc] = (float)v;
    }
  }
}

/* ---- DiT ---------------------------------------------------------------- */

/* DiT.forward (flow_reference.py:355-400) as assembled by build_dit /
 * dit_block (src/flow/dit.cpp:53-145). */
int orc_dit_forward(const orc_dit* w, int B, int T, const float* x, const float* mu,
                    const float* cond, const float* spks, const float* t, float* dphi,
                    const orc_dit_capture* cap) {
  const int D = w->dim, F = w->ff_inner, mel = w->mel_dim, H = w->heads, hd = w->head_dim;
  const long rows = (long)B * T;
  const int CIN = 4 * mel;
  float* temb = (float*)malloc(sizeof(float) * B * D);
  float* st = (float*)malloc(sizeof(float) * B * D);
  float* emb = (float*)malloc(sizeof(float) * B * 6 * D);
  float* A0 = (float*)malloc(sizeof(float) * rows * CIN);
  float* xe = (float*)malloc(sizeof(float) * rows * D);
  float* c1 = (float*)malloc(sizeof(float) * rows * D);
  float* c2 = (float*)malloc(sizeof(float) * rows * D);
  float* h = (float*)malloc(sizeof(float) * rows * D);
  float* xn = (float*)malloc(sizeof(float) * rows * D);
  float* q = (float*)malloc(sizeof(float) * rows * D);
  float* k = (float*)malloc(sizeof(float) * rows * D);
  float* v = (float*)malloc(sizeof(float) * rows * D);
  float* att = (float*)malloc(sizeof(float) * rows * D);
  float* y = (float*)malloc(sizeof(float) * rows * D);
  float* ff = (float*)malloc(sizeof(float) * rows * F);
  float* P = (float*)malloc(sizeof(float) * rows * mel);
  int* pos = (int*)malloc(sizeof(int) * T);
  if (!temb || !st || !emb || !A0 || !xe || !c1 || !c2 || !h || !xn || !q || !k || !v || !att ||
      !y || !ff || !P || !pos)
    return -4;
  for (int i = 0; i < T; ++i) pos[i] = i;

  /* time embedding (flow_matching.cpp:10-42) */
  orc_time_mlp(t, B, w->time_mlp_0_w, w->time_mlp_0_b, w->time_mlp_2_w, w->time_mlp_2_b, D, temb);
  if (cap && cap->time_embed) memcpy(cap->time_embed, temb, sizeof(float) * B * D);
  orc_silu_vec(temb, st, (long)B * D);

  /* InputEmbedding: proj(concat[x, cond, mu, spks]) (dit.cpp:109-110) */
  for (int b = 0; b < B; ++b)
    for (int tt = 0; tt < T; ++tt) {
      float* a = A0 + ((long)b * T + tt) * CIN;
      for (int c = 0; c < mel; ++c) {
        a[c] = x[((long)b * mel + c) * T + tt];
        a[mel + c] = cond[((long)b * mel + c) * T + tt];
        a[2 * mel + c] = mu[((long)b * mel + c) * T + tt];
        a[3 * mel + c] = spks[(long)b * mel + c];
      }
    }
  orc_linear(A0, CIN, w->input_proj_w, w->input_proj_b, xe, D, (int)rows, D, CIN);
  if (cap && cap->input_proj) memcpy(cap->input_proj, xe, sizeof(float) * rows * D);
  /* conv_pos_embed (dit.cpp:113-121) + residual (dit.cpp:122) */
  orc_conv_pos_mish(xe, w->conv_pos_1_w, w->conv_pos_1_b, NULL, c1, B, T, D, 16, 31);
  orc_conv_pos_mish(c1, w->conv_pos_2_w, w->conv_pos_2_b, NULL, c2, B, T, D, 16, 31);
  if (cap && cap->conv_pos) memcpy(cap->conv_pos, c2, sizeof(float) * rows * D);
  for (long i = 0; i < rows * D; ++i) h[i] = (float)((double)xe[i] + (double)c2[i]);
  if (cap && cap->input_embed) memcpy(cap->input_embed, h, sizeof(float) * rows * D);

  for (int bi = 0; bi < w->depth; ++bi) {
    const orc_dit_block* bw = &w->blocks[bi];
    /* emb = Linear(silu(t)), chunks shift/scale/gate msa, mlp (dit.cpp:56-62) */
    orc_linear(st, D, bw->attn_norm_w, bw->attn_norm_b, emb, 6 * D, B, 6 * D, D);
    const long es = 6 * D;
    orc_adaln(h, emb, emb + D, es, xn, B, T, D, 1e-6f);
    orc_linear(xn, D, bw->to_q_w, bw->to_q_b, q, D, (int)rows, D, D);
    orc_linear(xn, D, bw->to_k_w, bw->to_k_b, k, D, (int)rows, D, D);
    orc_linear(xn, D, bw->to_v_w, bw->to_v_b, v, D, (int)rows, D, D);
    orc_rope_partial(q, pos, B, T, D, 64, 10000.0f);
    orc_rope_partial(k, pos, B, T, D, 64, 10000.0f);
    orc_attention(q, D, k, D, v, D, att, D, B, T, T, H, H, hd, (float)(1.0 / sqrt((double)hd)), 0,
                  0);
    orc_linear(att, D, bw->to_out_w, bw->to_out_b, y, D, (int)rows, D, D);
    orc_gated_residual(h, y, emb + 2 * D, es, B, T, D);
    orc_adaln(h, emb + 3 * D, emb + 4 * D, es, xn, B, T, D, 1e-6f);
    orc_linear(xn, D, bw->ff0_w, bw->ff0_b, ff, F, (int)rows, F, D);
    orc_gelu_tanh(ff, ff, rows * F);
    orc_linear(ff, F, bw->ff2_w, bw->ff2_b, y, D, (int)rows, D, F);
    orc_gated_residual(h, y, emb + 5 * D, es, B, T, D);
    if (cap && cap->blocks) memcpy(cap->blocks + (long)bi * rows * D, h, sizeof(float) * rows * D);
  }
  /* norm_out: AdaLayerNormZero_Final, chunk order scale, shift (dit.cpp:133-136) */
  orc_linear(st, D, w->norm_out_w, w->norm_out_b, emb, 2 * D, B, 2 * D, D);
  orc_adaln(h, emb + D, emb, 2 * D, xn, B, T, D, 1e-6f);
  if (cap && cap->norm_out) memcpy(cap->norm_out, xn, sizeof(float) * rows * D);
  orc_linear(xn, D, w->proj_out_w, w->proj_out_b, P, mel, (int)rows, mel, D);
  for (int b = 0; b < B; ++b)
    for (int tt = 0; tt < T; ++tt)
      for (int c = 0; c < mel; ++c)
        dphi[((long)b * mel + c) * T + tt] = P[((long)b * T + tt) * mel + c];

  free(temb); free(st); free(emb); free(A0); free(xe); free(c1); free(c2); free(h); free(xn);
  free(q); free(k); free(v); free(att); free(y); free(ff); free(P); free(pos);
  return 0;
}

/* One Euler step with CFG (src/flow/flow.cpp:240-259). */
int orc_cfm_step(const orc_dit* w, int T, float* x, const float* mu, const float* cond,
                 const float* spks, float t, float dt, float cfg_rate) {
  const int mel = w->mel_dim;
  const long n = (long)mel * T;
  float* xin = (float*)calloc(2 * n, sizeof(float));
  float* muin = (float*)calloc(2 * n, sizeof(float));
  float* cin = (float*)calloc(2 * n, sizeof(float));
  float* sin_ = (float*)calloc(2 * mel, sizeof(float));
  float* dphi = (float*)malloc(sizeof(float) * 2 * n);
  if (!xin || !muin || !cin || !sin_ || !dphi) return -4;
  memcpy(xin, x, sizeof(float) * n);
  memcpy(xin + n, x, sizeof(float) * n);
  memcpy(muin, mu, sizeof(float) * n);
  memcpy(cin, cond, sizeof(float) * n);
  memcpy(sin_, spks, sizeof(float) * mel);
  const float tt[2] = {t, t};
  int rc = orc_dit_forward(w, 2, T, xin, muin, cin, sin_, tt, dphi, NULL);
  const float a = 1.0f + cfg_rate, b = cfg_rate;
  for (long i = 0; i < n; ++i) x[i] += dt * (a * dphi[i] - b * dphi[i + n]);
  free(xin); free(muin); free(cin); free(sin_); free(dphi);
  return rc;
}

/* solve_euler with t_span = 1 - cos(linspace(0,1,n+1) pi/2)
 * (src/flow/flow.cpp:202-274; flow_reference.py:468-501). */
int orc_cfm_solve(const orc_dit* w, int T, float* x, const float* mu, const float* cond,
                  const float* spks, int n_steps, float cfg_rate) {
  const float PI = 3.14159265358979323846f;
  float* ts = (float*)malloc(sizeof(float) * (n_steps + 1));
  for (int i = 0; i <= n_steps; ++i) {
    float u = (float)i / (float)n_steps;
    ts[i] = 1.0f - cosf(u * 0.5f * PI);
  }
  float t = ts[0], dt = ts[1] - ts[0];
  int rc = 0;
  for (int step = 1; step <= n_steps && rc == 0; ++step) {
    rc = orc_cfm_step(w, T, x, mu, cond, spks, t, dt, cfg_rate);
    t += dt;
    if (step < n_steps) dt = ts[step + 1] - t;
  }
  free(ts);
  return rc;
}

/* ---- Qwen2 --------------------------------------------------------------- */

/* Flow frontend, restating src/flow/flow.cpp:139-156 with
 *   l2_normalize  src/flow/ops.cpp:106-112 (x / sqrt(max(sum x^2, 1e-12))),
 *   PreLookahead  src/flow/prelookahead.cpp:8-20 (conv1 k=4 over the input
 *                 padded by 3 zeros on the right, leaky_relu slope 0.01,
 *                 conv2 k=3 over 2 zeros on the left, + input),
 *   repeat_interleave_2_ne0  src/flow/ops.cpp:114-122 (each token -> 2 frames),
 *   cond = ggml_pad(prompt_feat^T) (flow.cpp:155-156).
 * Convolutions accumulate in fp64; every stage is stored fp32. */
int orc_flow_frontend(const orc_flow_front* w, const int* ids, int Tseq, const float* prompt_feat,
                      int mel_len1, const float* spk_embedding, float* spk, float* token_embed,
                      float* pre, float* mu, float* cond) {
  const int mel = w->mel, ch = w->channels, K1 = 4, K2 = 3;
  for (int i = 0; i < Tseq; ++i)
    if (ids[i] < 0 || ids[i] >= w->vocab) return -3;
  /* speaker affine */
  double ss = 0.0;
  for (int k = 0; k < w->spk_in; ++k) ss += (double)spk_embedding[k] * spk_embedding[k];
  if (ss < 1e-12) ss = 1e-12;
  const double den = sqrt(ss);
  for (int o = 0; o < mel; ++o) {
    double acc = 0.0;
    for (int k = 0; k < w->spk_in; ++k)
      acc += (double)w->spk_affine_w[(long)o * w->spk_in + k] * (float)(spk_embedding[k] / den);
    spk[o] = (float)(acc + w->spk_affine_b[o]);
  }
  float* emb = (float*)malloc(sizeof(float) * (size_t)Tseq * mel);
  float* y1 = (float*)malloc(sizeof(float) * (size_t)Tseq * ch);
  float* h = (float*)malloc(sizeof(float) * (size_t)Tseq * mel);
  if (!emb || !y1 || !h) {
    free(emb);
    free(y1);
    free(h);
    return -4;
  }
  for (int t = 0; t < Tseq; ++t)
    memcpy(emb + (long)t * mel, w->input_embedding + (long)ids[t] * mel, sizeof(float) * mel);
  /* conv1: y1[t][oc] = b1[oc] + sum_{k<4, c} W1[oc][c][k] x[t + k][c] (x = 0 past T) */
#pragma omp parallel for schedule(static)
  for (int t = 0; t < Tseq; ++t) {
    for (int oc = 0; oc < ch; ++oc) {
      double acc = 0.0;
      for (int k = 0; k < K1; ++k) {
        const int src = t + k;
        if (src >= Tseq) continue;
        for (int c = 0; c < mel; ++c)
          acc += (double)w->pre_conv1_w[((long)oc * mel + c) * K1 + k] * emb[(long)src * mel + c];
      }
      const float v = (float)(acc + w->pre_conv1_b[oc]);
      y1[(long)t * ch + oc] = v > 0.0f ? v : 0.01f * v; /* leaky_relu(0.01) */
    }
  }
  /* conv2: h[t][oc] = b2[oc] + sum_{k<3, c} W2[oc][c][k] y1[t + k - 2][c] (0 before 0), + x */
#pragma omp parallel for schedule(static)
  for (int t = 0; t < Tseq; ++t) {
    for (int oc = 0; oc < mel; ++oc) {
      double acc = 0.0;
      for (int k = 0; k < K2; ++k) {
        const int src = t + k - (K2 - 1);
        if (src < 0) continue;
        for (int c = 0; c < ch; ++c)
          acc += (double)w->pre_conv2_w[((long)oc * ch + c) * K2 + k] * y1[(long)src * ch + c];
      }
      const float conv = (float)(acc + w->pre_conv2_b[oc]);
      h[(long)t * mel + oc] = conv + emb[(long)t * mel + oc];
    }
  }
  const int MT = 2 * Tseq;
  for (int c = 0; c < mel; ++c)
    for (int t = 0; t < MT; ++t) {
      mu[(long)c * MT + t] = h[(long)(t / 2) * mel + c];
      cond[(long)c * MT + t] = t < mel_len1 ? prompt_feat[(long)t * mel + c] : 0.0f;
    }
  if (token_embed) memcpy(token_embed, emb, sizeof(float) * (size_t)Tseq * mel);
  if (pre) memcpy(pre, h, sizeof(float) * (size_t)Tseq * mel);
  free(emb);
  free(y1);
  free(h);
  return 0;
}

int orc_qwen2_build_lm_input(const orc_qwen2* w, const int* text, int n_text, const int* speech,
                             int n_speech, float* out) {
  for (int i = 0; i < n_text; ++i)
    if (text[i] < 0 || text[i] >= w->text_vocab) return -3;
  for (int i = 0; i < n_speech; ++i)
    if (speech[i] < 0 || speech[i] >= w->speech_vocab) return -3;
  const int H = w->hidden;
  const int sos = 6561, task = 6563; /* src/llm/internal.h:33-34 */
  float* p = out;
  orc_embed_gather(w->speech_embedding, w->speech_vocab, H, &sos, 1, p);
  p += H;
  orc_embed_gather(w->embed_tokens, w->text_vocab, H, text, n_text, p);
  p += (long)n_text * H;
  orc_embed_gather(w->speech_embedding, w->speech_vocab, H, &task, 1, p);
  p += H;
  orc_embed_gather(w->speech_embedding, w->speech_vocab, H, speech, n_speech, p);
  return 1 + n_text + 1 + n_speech;
}

/* Qwen2 layer loop of prefill / decode (src/llm/llm.cpp:141-180, 254-299). */
int orc_qwen2_forward(const orc_qwen2* w, const float* x_in, int L, int past, float* k_cache,
                      float* v_cache, int cap, float* logits, float* hidden, float* final_norm) {
  const int H = w->hidden, I = w->intermediate, NH = w->n_heads, NKV = w->n_kv_heads,
            hd = w->head_dim;
  const int KV = NKV * hd;
  if (past + L > cap) return -5;
  float* x = (float*)malloc(sizeof(float) * L * H);
  float* hn = (float*)malloc(sizeof(float) * L * H);
  float* q = (float*)malloc(sizeof(float) * L * H);
  float* kk = (float*)malloc(sizeof(float) * L * KV);
  float* vv = (float*)malloc(sizeof(float) * L * KV);
  float* att = (float*)malloc(sizeof(float) * L * H);
  float* y = (float*)malloc(sizeof(float) * L * H);
  float* g = (float*)malloc(sizeof(float) * L * I);
  float* u = (float*)malloc(sizeof(float) * L * I);
  int* pos = (int*)malloc(sizeof(int) * L);
  if (!x || !hn || !q || !kk || !vv || !att || !y || !g || !u || !pos) return -4;
  memcpy(x, x_in, sizeof(float) * L * H);
  for (int i = 0; i < L; ++i) pos[i] = past + i;
  for (int l = 0; l < w->n_layers; ++l) {
    const orc_qwen2_layer* lw = &w->layers[l];
    float* kc = k_cache + (long)l * cap * KV;
    float* vc = v_cache + (long)l * cap * KV;
    orc_rmsnorm(x, lw->in_norm, hn, L, H, w->rms_eps);
    orc_linear(hn, H, lw->q_w, lw->q_b, q, H, L, H, H);
    orc_linear(hn, H, lw->k_w, lw->k_b, kk, KV, L, KV, H);
    orc_linear(hn, H, lw->v_w, lw->v_b, vv, KV, L, KV, H);
    orc_rope_neox(q, pos, L, NH, hd, H, w->rope_theta);
    orc_rope_neox(kk, pos, L, NKV, hd, KV, w->rope_theta);
    memcpy(kc + (long)past * KV, kk, sizeof(float) * L * KV);
    memcpy(vc + (long)past * KV, vv, sizeof(float) * L * KV);
    orc_attention(q, H, kc, KV, vc, KV, att, H, 1, L, past + L, NH, NKV, hd,
                  (float)(1.0 / sqrt((double)hd)), 1, past);
    orc_linear(att, H, lw->o_w, NULL, y, H, L, H, H);
    for (long i = 0; i < (long)L * H; ++i) x[i] = (float)((double)x[i] + (double)y[i]);
    orc_rmsnorm(x, lw->post_norm, hn, L, H, w->rms_eps);
    orc_linear(hn, H, lw->gate_w, NULL, g, I, L, I, H);
    orc_linear(hn, H, lw->up_w, NULL, u, I, L, I, H);
    orc_swiglu(g, u, g, (long)L * I);
    orc_linear(g, I, lw->down_w, NULL, y, H, L, H, I);
    for (long i = 0; i < (long)L * H; ++i) x[i] = (float)((double)x[i] + (double)y[i]);
    if (hidden) memcpy(hidden + (long)l * L * H, x, sizeof(float) * L * H);
  }
  orc_rmsnorm(x, w->final_norm, hn, L, H, w->rms_eps);
  if (final_norm) memcpy(final_norm, hn, sizeof(float) * L * H);
  if (logits) orc_linear(hn, H, w->llm_decoder, NULL, logits, w->speech_vocab, L, w->speech_vocab, H);
  free(x); free(hn); free(q); free(kk); free(vv); free(att); free(y); free(g); free(u); free(pos);
  return 0;
}
