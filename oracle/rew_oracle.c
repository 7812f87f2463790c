/*
 * rew_oracle.c -- CPU restatement of rew's eager op semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / the timed CPU column.  It is never part of the product path.
 *
 * The reference executes these ops inside the XLA CPU PJRT plugin
 * (gomlx/pjrt-cpu-binaries v0.104.0), which cannot be built or fetched here,
 * so this file restates the semantics from rew's sources (cited per
 * function, paths relative to the rew repository) and the StableHLO spec.
 *
 * Conventions:
 *  - float32 elementwise ops are single IEEE operations (bit-exact for
 *    + - * / max min sqrt, libm for transcendentals);
 *  - sums and dot products accumulate in double and round once to float
 *    (a high-precision reference for the implementation-defined reduction
 *    order of XLA);
 *  - bfloat16 values travel as uint16 bit patterns; a bf16 op computes in
 *    float and rounds to bf16 (RNE) at the op boundary.
 */
#include "rew_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* Threads the OpenMP loops below use (the cpu_baseline's core count). */
int orc_num_threads(void) { return omp_get_max_threads(); }

/* ---- rng: src/rew/rng.nim:32-80, src/rew/nn/init.nim:14-51 ------------------ */

static uint32_t rotl(uint32_t x, uint32_t r) { return (x << r) | (x >> (32u - r)); }

void orc_threefry(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1, uint32_t out[2]) {
  /* rng.nim:39-55: 4 rounds, rotations 13 15 26 6, parity 0x1BD11BDA */
  static const uint32_t R[4] = {13u, 15u, 26u, 6u};
  uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
  uint32_t x0 = c0 + k0, x1 = c1 + k1;
  for (int r = 0; r < 4; ++r) {
    x0 = x0 + x1;
    x1 = rotl(x1, R[r]);
    x1 = x1 ^ x0;
  }
  out[0] = x0 + k1;
  out[1] = x1 + k2 + 1u;
}

void orc_split(uint32_t k0, uint32_t k1, int n, uint32_t* out) {
  /* rng.nim:65-73: child i = threefry(k, (i, 0)) */
  for (int i = 0; i < n; ++i) orc_threefry(k0, k1, (uint32_t)i, 0u, out + 2 * i);
}

void orc_fold_in(uint32_t k0, uint32_t k1, uint64_t data, uint32_t out[2]) {
  /* rng.nim:75-80 */
  orc_threefry(k0, k1, (uint32_t)(data & 0xffffffffu), (uint32_t)(data >> 32), out);
}

static float unit24(uint32_t x) { return (float)(x >> 8) * (1.0f / 16777216.0f); }

void orc_uniform_f32(uint32_t k0, uint32_t k1, int64_t n, float lo, float hi, float* out) {
  /* init.nim:19-27 */
  float scale = hi - lo;
  for (int64_t i = 0; i < n; ++i) {
    uint32_t k[2];
    orc_fold_in(k0, k1, (uint64_t)i, k);
    out[i] = lo + scale * unit24(k[0]);
  }
}

void orc_normal_f32(uint32_t k0, uint32_t k1, int64_t n, float mean, float sd, float* out) {
  /* init.nim:29-51: Box-Muller on pairs, u1 clamped to >= 1e-10 */
  int64_t pairs = (n + 1) / 2;
  float two_pi = 2.0f * (float)3.14159265358979323846;
  for (int64_t i = 0; i < pairs; ++i) {
    uint32_t a[2], b[2];
    orc_fold_in(k0, k1, (uint64_t)(2 * i), a);
    orc_fold_in(k0, k1, (uint64_t)(2 * i + 1), b);
    float u1 = unit24(a[0]), u2 = unit24(b[0]);
    float su1 = u1 > 1e-10f ? u1 : 1e-10f;
    float r = sqrtf(-2.0f * logf(su1));
    float th = two_pi * u2;
    float z0 = r * cosf(th), z1 = r * sinf(th);
    out[2 * i] = mean + sd * z0;
    if (2 * i + 1 < n) out[2 * i + 1] = mean + sd * z1;
  }
}

/* ---- bf16 ------------------------------------------------------------------- */

uint16_t orc_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float rbf(float f) { return orc_bf16_f32(orc_bf16(f)); }

void orc_f32_to_bf16(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16(x[i]);
}

void orc_bf16_to_f32(const uint16_t* x, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_f32(x[i]);
}

/* ---- elementwise float32 (StableHLO semantics) -------------------------------- */

/* IEEE 754-2019 maximum / minimum: NaN propagates, -0 < +0. */
static float fmax_prop(float a, float b) {
  if (a != a || b != b) return NAN;
  if (a == b) return signbit(a) ? b : a;
  return a > b ? a : b;
}
static float fmin_prop(float a, float b) {
  if (a != a || b != b) return NAN;
  if (a == b) return signbit(a) ? a : b;
  return a < b ? a : b;
}

float orc_binary_scalar(int op, float a, float b) {
  switch (op) {
    case ORC_ADD: return a + b;
    case ORC_SUB: return a - b;
    case ORC_MUL: return a * b;
    case ORC_DIV: return a / b;
    case ORC_MAX: return fmax_prop(a, b);
    case ORC_MIN: return fmin_prop(a, b);
    case ORC_POW: return powf(a, b);
    case ORC_REM: return fmodf(a, b);
    case ORC_ATAN2: return atan2f(a, b);
    default: return NAN;
  }
}

void orc_binary_f32(int op, const float* a, const float* b, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_binary_scalar(op, a[i], b[i]);
}

float orc_unary_scalar(int op, float x) {
  switch (op) {
    case ORC_NEG: return -x;
    case ORC_ABS: return fabsf(x);
    case ORC_EXP: return expf(x);
    case ORC_LOG: return logf(x);
    case ORC_SQRT: return sqrtf(x);
    case ORC_RSQRT: return 1.0f / sqrtf(x);
    case ORC_TANH: return tanhf(x);
    case ORC_LOGISTIC: return 1.0f / (1.0f + expf(-x));
    case ORC_SIN: return sinf(x);
    case ORC_COS: return cosf(x);
    case ORC_FLOOR: return floorf(x);
    case ORC_CEIL: return ceilf(x);
    default: return NAN;
  }
}

void orc_unary_f32(int op, const float* a, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_unary_scalar(op, a[i]);
}

/* ---- reductions: src/rew/eager.nim:1027-1057, stablehlo/ops.nim:2005-2057 ----- */

void orc_reduce_f32(int op, const float* x, int rank, const int64_t* shape, int ndims,
                    const int64_t* dims, float* out) {
  int red[16] = {0};
  for (int i = 0; i < ndims; ++i) red[dims[i]] = 1;
  int64_t stride[16];
  int64_t acc = 1;
  for (int i = rank - 1; i >= 0; --i) {
    stride[i] = acc;
    acc *= shape[i];
  }
  int64_t n_out = 1, n_red = 1;
  int kept[16], rd[16], nk = 0, nr = 0;
  for (int i = 0; i < rank; ++i) {
    if (red[i]) { rd[nr++] = i; n_red *= shape[i]; }
    else { kept[nk++] = i; n_out *= shape[i]; }
  }
  for (int64_t o = 0; o < n_out; ++o) {
    int64_t base = 0, t = o;
    for (int j = nk - 1; j >= 0; --j) {
      base += (t % shape[kept[j]]) * stride[kept[j]];
      t /= shape[kept[j]];
    }
    double s = (op == ORC_RPROD) ? 1.0 : 0.0;
    float m = (op == ORC_RMAX) ? -INFINITY : INFINITY;
    for (int64_t r = 0; r < n_red; ++r) {
      int64_t off = base, u = r;
      for (int j = nr - 1; j >= 0; --j) {
        off += (u % shape[rd[j]]) * stride[rd[j]];
        u /= shape[rd[j]];
      }
      float v = x[off];
      switch (op) {
        case ORC_RSUM: s += v; break;
        case ORC_RPROD: s *= v; break;
        case ORC_RMAX: m = fmax_prop(m, v); break;
        default: m = fmin_prop(m, v); break;
      }
    }
    out[o] = (op == ORC_RSUM || op == ORC_RPROD) ? (float)s : m;
  }
}

/* ---- dot_general: src/rew/eager.nim:1000-1014, stablehlo/ops.nim:1813-1908 ---- */

static double load_elem(int dt, const void* p, int64_t i) {
  if (dt == ORC_BF16) return (double)orc_bf16_f32(((const uint16_t*)p)[i]);
  return (double)((const float*)p)[i];
}

void orc_dot_general(int dt, const void* a, int ra, const int64_t* sa, const void* b, int rb,
                     const int64_t* sb, int nbatch, const int64_t* lb, const int64_t* rbd,
                     int ncon, const int64_t* lc, const int64_t* rc, void* out) {
  int ua[16] = {0}, ub[16] = {0};
  for (int i = 0; i < nbatch; ++i) { ua[lb[i]] = 1; ub[rbd[i]] = 1; }
  for (int i = 0; i < ncon; ++i) { ua[lc[i]] = 1; ub[rc[i]] = 1; }
  int fa[16], fb[16], nfa = 0, nfb = 0;
  for (int i = 0; i < ra; ++i) if (!ua[i]) fa[nfa++] = i;
  for (int i = 0; i < rb; ++i) if (!ub[i]) fb[nfb++] = i;
  int64_t sta[16], stb[16], acc = 1;
  for (int i = ra - 1; i >= 0; --i) { sta[i] = acc; acc *= sa[i]; }
  acc = 1;
  for (int i = rb - 1; i >= 0; --i) { stb[i] = acc; acc *= sb[i]; }
  int64_t NB = 1, M = 1, N = 1, K = 1;
  for (int i = 0; i < nbatch; ++i) NB *= sa[lb[i]];
  for (int i = 0; i < nfa; ++i) M *= sa[fa[i]];
  for (int i = 0; i < nfb; ++i) N *= sb[fb[i]];
  for (int i = 0; i < ncon; ++i) K *= sa[lc[i]];
  int64_t* ka = (int64_t*)malloc(sizeof(int64_t) * (size_t)(K ? K : 1));
  int64_t* kb = (int64_t*)malloc(sizeof(int64_t) * (size_t)(K ? K : 1));
  for (int64_t k = 0; k < K; ++k) {
    int64_t oa = 0, ob = 0, t = k;
    for (int j = ncon - 1; j >= 0; --j) {
      int64_t c = t % sa[lc[j]];
      t /= sa[lc[j]];
      oa += c * sta[lc[j]];
      ob += c * stb[rc[j]];
    }
    ka[k] = oa;
    kb[k] = ob;
  }
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int64_t bi = 0; bi < NB; ++bi) {
    for (int64_t m = 0; m < M; ++m) {
      int64_t oa = 0, obb = 0, t = bi;
      for (int j = nbatch - 1; j >= 0; --j) {
        int64_t c = t % sa[lb[j]];
        t /= sa[lb[j]];
        oa += c * sta[lb[j]];
        obb += c * stb[rbd[j]];
      }
      t = m;
      for (int j = nfa - 1; j >= 0; --j) {
        oa += (t % sa[fa[j]]) * sta[fa[j]];
        t /= sa[fa[j]];
      }
      for (int64_t n = 0; n < N; ++n) {
        int64_t ob = obb, u = n;
        for (int j = nfb - 1; j >= 0; --j) {
          ob += (u % sb[fb[j]]) * stb[fb[j]];
          u /= sb[fb[j]];
        }
        double s = 0.0;
        for (int64_t k = 0; k < K; ++k) s += load_elem(dt, a, oa + ka[k]) * load_elem(dt, b, ob + kb[k]);
        int64_t o = (bi * M + m) * N + n;
        if (dt == ORC_BF16) ((uint16_t*)out)[o] = orc_bf16((float)s);
        else ((float*)out)[o] = (float)s;
      }
    }
  }
  free(ka);
  free(kb);
}

/* Dense row-major GEMM fast path: C[M,N] = A[M,K] B[K,N], float operands,
 * double accumulation, optional bf16 rounding of the result. */
void orc_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
              int round_bf16) {
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)N);
#pragma omp for schedule(dynamic, 1)
    for (int64_t m = 0; m < M; ++m) {
      for (int64_t n = 0; n < N; ++n) acc[n] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double av = (double)A[m * K + k];
        const float* brow = B + k * N;
        for (int64_t n = 0; n < N; ++n) acc[n] += av * (double)brow[n];
      }
      for (int64_t n = 0; n < N; ++n) {
        float v = (float)acc[n];
        C[m * N + n] = round_bf16 ? rbf(v) : v;
      }
    }
    free(acc);
  }
}

/* ---- composites ------------------------------------------------------------ */

/* softmax over the last axis: src/rew/nn/activation.nim:64-77 */
void orc_softmax_rows(const float* x, int64_t rows, int64_t cols, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* orow = out + r * cols;
    float m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) m = fmax_prop(m, xr[c]);
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      orow[c] = expf(xr[c] - m);
      s += orow[c];
    }
    float sf = (float)s;
    for (int64_t c = 0; c < cols; ++c) orow[c] = orow[c] / sf;
  }
}

/* rmsNorm: src/rew/nn/norm.nim:204-224 -- gamma * (x / sqrt(mean(x^2) + eps)) */
void orc_rmsnorm_rows(const float* x, const float* gamma, int64_t rows, int64_t cols, float eps,
                      float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += (double)(xr[c] * xr[c]);
    float meanSq = (float)s / (float)cols;
    float rms = sqrtf(meanSq + eps);
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = gamma[c] * (xr[c] / rms);
  }
}

/* LayerNorm.forward over the last axis: src/rew/nn/norm.nim:41-84 */
void orc_layernorm_rows(const float* x, const float* gamma, const float* beta, int64_t rows,
                        int64_t cols, float eps, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += xr[c];
    float mean = (float)s / (float)cols;
    double v = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      float d = xr[c] - mean;
      v += (double)(d * d);
    }
    float var = (float)v / (float)cols;
    float inv = 1.0f / sqrtf(var + eps);
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = gamma[c] * ((xr[c] - mean) * inv) + beta[c];
  }
}

/* RoPE on adjacent pairs: src/rew/nn/rope.nim:56-108, 153-179.
 * x: [outer, S, D] float; tables [maxSeq, D] with entries duplicated at
 * (2i, 2i+1); rows offset..offset+S are used. */
void orc_rope(const float* x, const float* cos_t, const float* sin_t, int64_t outer, int64_t S,
              int64_t D, int64_t offset, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t s = 0; s < S; ++s) {
      const float* xr = x + (o * S + s) * D;
      const float* cr = cos_t + (offset + s) * D;
      const float* sr = sin_t + (offset + s) * D;
      float* orow = out + (o * S + s) * D;
      for (int64_t i = 0; i < D / 2; ++i) {
        float x0 = xr[2 * i], x1 = xr[2 * i + 1];
        float c = cr[2 * i], sn = sr[2 * i];
        orow[2 * i] = c * x0 - sn * x1;
        orow[2 * i + 1] = sn * x0 + c * x1;
      }
    }
}

/* scaledDotProductAttention with GQA head sharing: src/rew/nn/attention.nim:36-81,
 * groupedqueryattention.nim:126-133 (kv head = h / (H / Hkv)).
 * q [B,H,Sq,D], k/v [B,Hkv,Sk,D]; causal = 1 uses makeCausalMask's orientation
 * (attention.nim:18-34): score[i][j] gets -1e9 where i > j; causal = 2 is the
 * mirrored mask (-1e9 where i < j); 0 is unmasked.
 * mixed = 1 emulates the bf16 op sequence: q/k/v are bf16-valued, scores
 * are rounded to bf16 before the fp32 scale/mask/softmax, probabilities are
 * rounded to bf16 before the PV product, the output is rounded to bf16. */
void orc_sdpa(const float* q, const float* k, const float* v, int64_t B, int64_t H,
              int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, int causal, float scale, int mixed,
              float* out) {
  const int64_t g = H / Hkv;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t hk = h / g;
      float* p = (float*)malloc(sizeof(float) * (size_t)Sk);
      for (int64_t i = 0; i < Sq; ++i) {
        const float* qi = q + ((b * H + h) * Sq + i) * D;
        for (int64_t j = 0; j < Sk; ++j) {
          const float* kj = k + ((b * Hkv + hk) * Sk + j) * D;
          double s = 0.0;
          for (int64_t d = 0; d < D; ++d) s += (double)qi[d] * (double)kj[d];
          float sf = (float)s;
          if (mixed) sf = rbf(sf);
          sf = sf * scale;
          if (causal == 1) sf = sf + ((i <= j) ? 0.0f : -1e9f);
          else if (causal == 2) sf = sf + ((i >= j) ? 0.0f : -1e9f);
          else if (causal == 3) sf = sf + ((i < j) ? 0.0f : -1e9f);
          else if (causal == 4) sf = sf + ((i > j) ? 0.0f : -1e9f);
          p[j] = sf;
        }
        float m = -INFINITY;
        for (int64_t j = 0; j < Sk; ++j) m = fmax_prop(m, p[j]);
        double sum = 0.0;
        for (int64_t j = 0; j < Sk; ++j) {
          p[j] = expf(p[j] - m);
          sum += p[j];
        }
        float sumf = (float)sum;
        for (int64_t j = 0; j < Sk; ++j) {
          p[j] = p[j] / sumf;
          if (mixed) p[j] = rbf(p[j]);
        }
        float* oi = out + ((b * H + h) * Sq + i) * D;
        for (int64_t d = 0; d < D; ++d) {
          double s = 0.0;
          for (int64_t j = 0; j < Sk; ++j) s += (double)p[j] * (double)v[((b * Hkv + hk) * Sk + j) * D + d];
          oi[d] = mixed ? rbf((float)s) : (float)s;
        }
      }
      free(p);
    }
}

/* argmax over the last axis with rew's composite semantics
 * (src/rew/ops/reduce.nim:202-225): first index of the max; a row holding a
 * NaN compares unequal everywhere and yields int32.high. */
void orc_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) m = fmax_prop(m, xr[c]);
    int32_t best = 2147483647;
    for (int64_t c = 0; c < cols; ++c)
      if (xr[c] == m) { best = (int32_t)c; break; }
    out[r] = best;
  }
}

/* topK over the last axis, largest first, ties to the lower index
 * (src/rew/ops/sort.nim:36-90 with a stable GE sort); NaN ranks below every
 * number. */
void orc_topk_rows(const float* x, int64_t rows, int64_t cols, int64_t k, float* vals,
                   int32_t* idx) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    unsigned char* taken = (unsigned char*)calloc((size_t)cols, 1);
    for (int64_t t = 0; t < k; ++t) {
      int64_t best = -1;
      for (int64_t c = 0; c < cols; ++c) {
        if (taken[c]) continue;
        if (best < 0) { best = c; continue; }
        float a = xr[c], bv = xr[best];
        int a_nan = a != a, b_nan = bv != bv;
        if (b_nan && !a_nan) best = c;
        else if (!a_nan && !b_nan && a > bv) best = c;
      }
      taken[best] = 1;
      vals[r * k + t] = xr[best];
      idx[r * k + t] = (int32_t)best;
    }
    free(taken);
  }
}
