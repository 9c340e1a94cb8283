/*
 * CPU oracle for the Bigger Bird v3 hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or the timed CPU baseline); the product path never calls it.
 *
 * What each function restates (paths relative to the reference repository):
 *   orc_routes      modal_rd/attention.py:143-174 (RDAttention.routes), under the deterministic arithmetic
 *                   contract below, which the HIP router reproduces bit for bit.
 *   orc_attn_rows   kernels/bigger_bird_flash_ref.py:10-52 and kernels/bigger_bird_flash.py:56-96 (union mask
 *                   front | causal window | routed, GQA head map, OFFSET = N - T), one query row at a time in
 *                   float64 so that 128K-token shapes can be checked on sampled rows; bf16 or fp16 elements
 *                   (kernels/bigger_bird_flash.py:110 accepts both).
 *   orc_quantize    modal_rd/kv_int8.py:19-22 (per-row symmetric int8, fp32 scale clamp_min 1e-4, RNE).
 *   orc_dequantize  modal_rd/kv_int8.py:25-26.
 *   orc_decode      modal_rd/attention.py:137-141 over the dequantised cache (exact attention of one token).
 *
 * Routing arithmetic contract.  The reference computes scores with a bf16 matmul (modal_rd/attention.py:164) whose
 * fp32 accumulation order is the library's; on the CPU that produced the golden routes (torch 2.10, oneDNN, AMX-BF16)
 * that order is fixed and reproduced exactly by amx_dot() below.  Every later step is fixed here as well:
 *   s    = bf16_rne(amx_dot(q, k))                     d even; score mode 1 uses bf16_rne(exact q.k) instead
 *          fp16_rne(f16_seq_dot(q, k))               fp16 q and k: torch's CPU fp16 matmul, one sequential fp32 chain
 *   x    = fp32(s * scaling)
 *   M_i  = max_j x_ij over causal keys j <= qpos_i
 *   e_ij = det_exp2(fp32(fp32(x_ij - M_i) * LOG2E))    det_exp2: rint reduction + degree-7 Horner with fmaf
 *   Z_i  = sum_j floor(e_ij * 2^40)                    uint64 fixed point, order independent
 *   p_ij = fp32(e_ij * fp32(2^40 / double(Z_i)))
 *   P_j  = sum_i floor(p_ij * 2^40)  (mean pool)  or  max_i floor(p_ij * 2^40)  (max pool)
 *   eligible j in [sink, n - window); take `budget` largest P_j, ties to the lower index; return ascending.
 * The bf16 scores are therefore bit-identical to the reference's; the softmax and mean differ from torch's fp32 ones by
 * a few fp32 ulps, which changes a selected column only where two pooled probabilities tie to that precision.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LOG2E_F 1.44269504088896340736f

/* Planted mistakes for the pinning tests (0 = none): 1 window edge off by one, 2 transposed GQA head map,
 * 3 routed keys ignore causality, 4 route ties to the higher index, 5 sink columns eligible for routing. */
static int g_mut = 0;
void orc_set_mutation(int m) { g_mut = m; }
#define FIX_ONE 1099511627776.0f /* 2^40 */

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}


/* IEEE binary16 conversions written out (gcc on x86 lacks _Float16 without AVX512-FP16). */
static inline float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff, u;
  if (exp == 0) {
    float f = ldexpf((float)man, -24); /* subnormal (or zero): exact */
    return sign ? -f : f;
  }
  if (exp == 31) u = sign | 0x7f800000u | (man << 13);
  else u = sign | ((exp + 112) << 23) | (man << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_f16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  float a = fabsf(f);
  if (isnan(f)) return sign | 0x7e00u;
  if (a >= 65520.0f) return sign | 0x7c00u; /* rounds to inf */
  if (a < 0x1p-14f) {                         /* fp16 subnormal range: spacing 2^-24, exact scaling then RNE */
    float m = nearbyintf(a * 0x1p24f);
    return sign | (uint16_t)m;                /* m == 1024 lands on the smallest normal, still correct bits */
  }
  uint32_t au;
  memcpy(&au, &a, 4);
  uint32_t rounded = au + 0xfffu + ((au >> 13) & 1u);
  rounded &= ~0x1fffu;
  uint32_t exp = (rounded >> 23) - 112;
  return sign | (uint16_t)((exp << 10) | ((rounded >> 13) & 0x3ff));
}

static inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint16_t orc_f32_to_f16(float f) { return f32_to_f16_rne(f); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* One round-to-nearest-even step from float64 straight to bf16 (no intermediate fp32 rounding). */
uint16_t orc_bf16_from_double(double x) {
  if (x == 0.0 || isnan(x) || isinf(x)) return f32_to_bf16_rne((float)x);
  double ax = fabs(x);
  double quantum;
  if (ax < 0x1p-126) {
    quantum = 0x1p-133; /* bf16 subnormal spacing */
  } else {
    int e;
    frexp(ax, &e);          /* ax = m * 2^e, m in [0.5, 1) */
    quantum = ldexp(1.0, e - 8);
  }
  double r = nearbyint(x / quantum) * quantum; /* exact scaling, RNE */
  float f = (float)r;                           /* exact: r has <= 8 significant bits (or overflows to inf) */
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)(u >> 16);
}

float orc_det_exp2(float x) {
  if (!(x > -100.0f)) return 0.0f;
  float n = rintf(x);
  float f = x - n;
  float p = 1.5252733804059840e-05f;
  p = fmaf(p, f, 1.5403530393381610e-04f);
  p = fmaf(p, f, 1.3333558146428443e-03f);
  p = fmaf(p, f, 9.6181291076284772e-03f);
  p = fmaf(p, f, 5.5504108664821580e-02f);
  p = fmaf(p, f, 2.4022650695910071e-01f);
  p = fmaf(p, f, 6.9314718055994531e-01f);
  p = fmaf(p, f, 1.0f);
  return ldexpf(p, (int)n);
}

static inline uint64_t fix40(float v) { return (uint64_t)(v * FIX_ONE); }

/*
 * fp32 score of one query row against one key row in the accumulation order of torch's CPU bf16 matmul on an
 * AMX-BF16 host (oneDNN brgemm, one tile dot-product per 32 elements of d): inside each 32-element block the even and
 * the odd elements form two sequential fp32 chains E and O; the block adds fl(E + O) to the running sum. A bf16 x bf16
 * product is exact in fp32, so every step is one fp32 rounding. (Pinned against torch.matmul on bf16 CPU tensors.)
 */
static inline float amx_dot(const uint16_t* a, const uint16_t* b, int d) {
  float acc = 0.0f;
  for (int b0 = 0; b0 < d; b0 += 32) {
    float e = 0.0f, o = 0.0f;
    for (int i = b0; i < b0 + 32 && i < d; i += 2) {
      e = e + bf16_to_f32(a[i]) * bf16_to_f32(b[i]);
      o = o + bf16_to_f32(a[i + 1]) * bf16_to_f32(b[i + 1]);
    }
    acc = acc + (e + o);
  }
  return acc;
}

/*
 * fp32 score of one query row against one key row for fp16 inputs, in the accumulation order of torch's CPU fp16
 * matmul (the reference's modal_rd/attention.py:164 on fp16 tensors): one sequential fp32 chain over d in order. An
 * fp16 x fp16 product is exact in fp32, so every step is one fp32 rounding. (Pinned against torch.matmul on fp16 CPU
 * tensors.)
 */
static inline float f16_seq_dot(const uint16_t* a, const uint16_t* b, int d) {
  float acc = 0.0f;
  for (int i = 0; i < d; ++i) acc = acc + f16_to_f32(a[i]) * f16_to_f32(b[i]);
  return acc;
}

/* fp32 -> the nearest fp16 value (ties to even), returned as fp32 (exact): 11 significant bits, subnormal spacing
 * 2^-24, magnitudes from 65520 up rounding to infinity. */
static inline float f16_round(float x) {
  if (x == 0.0f || isnan(x) || isinf(x)) return x;
  double ax = fabs((double)x);
  double quantum;
  if (ax < 0x1p-14) {
    quantum = 0x1p-24;
  } else {
    int e;
    frexp(ax, &e); /* ax = m * 2^e, m in [0.5, 1) */
    quantum = ldexp(1.0, e - 11);
  }
  double r = nearbyint((double)x / quantum) * quantum;
  if (fabs(r) > 65504.0) r = copysign(INFINITY, r);
  return (float)r;
}
float orc_f16_round(float x) { return f16_round(x); }
float orc_f16_dot(const uint16_t* a, const uint16_t* b, int d) { return f16_seq_dot(a, b, d); }

/* Exact float64 dot product (bf16 inputs, d <= 128: every partial sum is exact). */
static inline double exact_dot(const uint16_t* a, const uint16_t* b, int d) {
  double s = 0.0;
  for (int i = 0; i < d; ++i) s += (double)bf16_to_f32(a[i]) * (double)bf16_to_f32(b[i]);
  return s;
}

/* Score rounding of the routing contract: 0 = torch CPU AMX order (the reference's arithmetic), 1 = exact. */
static int g_score_mode = 0;
void orc_set_score_mode(int m) { g_score_mode = m; }
float orc_amx_dot(const uint16_t* a, const uint16_t* b, int d) { return amx_dot(a, b, d); }

/*
 * Pooled routing scores and the selected columns.
 *   q     bf16, element (h, t, c) at q[h*sq0 + t*sq1 + c]     (h in [0,H), t in [0,n) key-aligned positions)
 *   k     bf16, element (g, t, c) at k[g*sk0 + t*sk1 + c]
 *   qpos  r absolute query positions (ascending or not); causal: keys j <= qpos[i]
 *   pooled_out [H][n] uint64 (may be NULL); idx_out [H][budget] int32 ascending (may be NULL when budget == 0)
 * Returns 0, or a negative code on bad arguments.
 */
int orc_routes(const uint16_t* q, int64_t sq0, int64_t sq1, const uint16_t* k, int64_t sk0, int64_t sk1,
               int H, int Hkv, int n, int d, const int64_t* qpos, int r, int sink, int window, int budget,
               float scaling, int pool_max, uint64_t* pooled_out, int32_t* idx_out, int nthreads, int is_f16) {
  if (H <= 0 || Hkv <= 0 || H % Hkv || n <= 0 || d <= 0 || r <= 0 || budget < 0) return -1;
  int G = H / Hkv;
  int lo = sink < n ? (sink < 0 ? 0 : sink) : n;
  if (g_mut == 5) lo = 0;
  int hi = n - window;
  if (hi > n) hi = n;
  int eligible = hi > lo ? hi - lo : 0;
  if (budget > eligible) return -2;
  uint64_t* pooled = pooled_out ? pooled_out : (uint64_t*)calloc((size_t)H * n, sizeof(uint64_t));
  if (!pooled) return -3;
  int err = 0;
  int nt = 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
  nt = omp_get_max_threads();
#endif
  float* xbuf = (float*)malloc(sizeof(float) * (size_t)n * nt);
  float* ebuf = (float*)malloc(sizeof(float) * (size_t)n * nt);
  if (!xbuf || !ebuf) {
    free(xbuf);
    free(ebuf);
    if (!pooled_out) free(pooled);
    return -3;
  }
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int h = 0; h < H; ++h) {
    int tid = 0;
#ifdef _OPENMP
    tid = omp_get_thread_num();
#endif
    float* x = xbuf + (size_t)tid * n;
    float* e = ebuf + (size_t)tid * n;
    int g = h / G;
    uint64_t* P = pooled + (size_t)h * n;
    memset(P, 0, sizeof(uint64_t) * (size_t)n);
    for (int i = 0; i < r; ++i) {
      int64_t qp = qpos[i];
      int last = qp < n - 1 ? (int)qp : n - 1; /* keys 0..last are causal */
      const uint16_t* qrow = q + h * sq0 + qp * sq1;
      float m = -INFINITY;
      for (int j = 0; j <= last; ++j) {
        const uint16_t* krow = k + g * sk0 + (int64_t)j * sk1;
        float sv;
        if (is_f16) {
          sv = f16_round(f16_seq_dot(qrow, krow, d));
        } else {
          uint16_t sb = g_score_mode ? orc_bf16_from_double(exact_dot(qrow, krow, d))
                                     : f32_to_bf16_rne(amx_dot(qrow, krow, d));
          sv = bf16_to_f32(sb);
        }
        float xv = sv * scaling;
        x[j] = xv;
        if (xv > m) m = xv;
      }
      uint64_t Z = 0;
      for (int j = 0; j <= last; ++j) {
        float t = (x[j] - m) * LOG2E_F;
        e[j] = orc_det_exp2(t);
        Z += fix40(e[j]);
      }
      float invz = (float)(1099511627776.0 / (double)Z);
      for (int j = 0; j <= last; ++j) {
        uint64_t pf = fix40(e[j] * invz);
        if (pool_max) {
          if (pf > P[j]) P[j] = pf;
        } else {
          P[j] += pf;
        }
      }
    }
  }
  free(xbuf);
  free(ebuf);
  if (idx_out && budget > 0) {
    /* Selection: budget largest pooled values among eligible columns, ties to the lower index, ascending output. */
    for (int h = 0; h < H; ++h) {
      const uint64_t* P = pooled + (size_t)h * n;
      /* threshold = budget-th largest value (order statistic via counting on a sorted copy) */
      uint64_t* vals = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)eligible);
      if (!vals) { err = -3; break; }
      memcpy(vals, P + lo, sizeof(uint64_t) * (size_t)eligible);
      /* partial selection: nth_element by simple quickselect (descending) */
      int64_t left = 0, right = eligible - 1, kth = budget - 1;
      while (left < right) {
        uint64_t pivot = vals[(left + right) / 2];
        int64_t a = left, b = right;
        while (a <= b) {
          while (vals[a] > pivot) ++a;
          while (vals[b] < pivot) --b;
          if (a <= b) { uint64_t t = vals[a]; vals[a] = vals[b]; vals[b] = t; ++a; --b; }
        }
        if (kth <= b) right = b; else if (kth >= a) left = a; else break;
      }
      uint64_t thr = vals[kth];
      free(vals);
      int above = 0;
      for (int j = lo; j < hi; ++j) above += P[j] > thr;
      int take_eq = budget - above, out = 0;
      int32_t* dst = idx_out + (size_t)h * budget;
      if (g_mut == 4) { /* planted mistake: ties resolved toward higher indices */
        int eq_total = 0;
        for (int j = lo; j < hi; ++j) eq_total += P[j] == thr;
        int skip = eq_total - take_eq;
        for (int j = lo; j < hi; ++j) {
          if (P[j] > thr) dst[out++] = j;
          else if (P[j] == thr) { if (skip > 0) --skip; else dst[out++] = j; }
        }
        continue;
      }
      for (int j = lo; j < hi; ++j) {
        if (P[j] > thr) dst[out++] = j;
        else if (P[j] == thr && take_eq > 0) { dst[out++] = j; --take_eq; }
      }
    }
  }
  if (!pooled_out) free(pooled);
  return err;
}

/*
 * float64 attention of selected query rows over the union mask.
 *   q [BH, T, D] (strides sq0, sq1), k/v [BH/kv_groups, N, D] (strides), idx [BH, NG, KR] (strides, -1 = none)
 *   key_mask [B, N] (uint8, may be NULL; stride smb per batch), rows: nrows pairs (bh, t) with t a local row.
 *   out [nrows, D] float64.
 */
int orc_attn_rows(const uint16_t* q, int64_t sq0, int64_t sq1, const uint16_t* k, int64_t sk0, int64_t sk1,
                  const uint16_t* v, int64_t sv0, int64_t sv1, const int32_t* idx, int64_t si0, int64_t si1,
                  int64_t si2, int NG, int KR, const uint8_t* key_mask, int64_t smb, int BH, int T, int N, int D,
                  int num_heads, int kv_groups, int front, int window, int64_t route_chunk, double scale,
                  const int64_t* rows, int nrows, double* out, int nthreads, int f16) {
  if (T > N || num_heads % kv_groups || BH % num_heads) return -1;
  float (*const elem)(uint16_t) = f16 ? f16_to_f32 : bf16_to_f32; /* q, k, v element type */
  if (front > N) front = N;
  int64_t offset = (int64_t)N - T;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
  int err = 0;
#ifdef _OPENMP
#pragma omp parallel
#endif
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)N);
    uint8_t* use = (uint8_t*)malloc((size_t)N);
    if (!s || !use) err = -3;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
    for (int rr = 0; rr < nrows; ++rr) {
      if (!s || !use) continue;
      int64_t bh = rows[2 * rr], t = rows[2 * rr + 1];
      int64_t qabs = t + offset;
      int64_t b = bh / num_heads;
      int64_t kvh = b * (num_heads / kv_groups) + (bh % num_heads) / kv_groups;
      if (g_mut == 2) kvh = b * (num_heads / kv_groups) + (bh % num_heads) % (num_heads / kv_groups);
      int64_t grp = qabs / route_chunk;
      if (grp >= NG) grp = NG - 1;
      memset(use, 0, (size_t)N);
      const int64_t wedge = g_mut == 1 ? qabs - window - 1 : qabs - window;
      for (int64_t j = 0; j <= qabs && j < N; ++j)
        if (j < front || j > wedge) use[j] = 1;
      for (int sl = 0; sl < KR; ++sl) {
        int64_t j = idx[bh * si0 + grp * si1 + sl * si2];
        if (g_mut == 3 ? (j >= front && j < N) : (j >= front && j <= qabs && j < qabs - window + 1 && j < N))
          use[j] = 1;
      }
      if (key_mask)
        for (int64_t j = 0; j < N; ++j) use[j] &= key_mask[b * smb + j] != 0;
      double mx = -INFINITY;
      const uint16_t* qr = q + bh * sq0 + t * sq1;
      for (int64_t j = 0; j < N; ++j) {
        if (!use[j]) continue;
        double acc = 0;
        const uint16_t* kr = k + kvh * sk0 + j * sk1;
        for (int c = 0; c < D; ++c) acc += (double)elem(qr[c]) * (double)elem(kr[c]);
        s[j] = acc * scale;
        if (s[j] > mx) mx = s[j];
      }
      double* o = out + (size_t)rr * D;
      for (int c = 0; c < D; ++c) o[c] = 0.0;
      if (mx == -INFINITY) continue; /* fully masked row -> 0 */
      double den = 0;
      for (int64_t j = 0; j < N; ++j) {
        if (!use[j]) continue;
        double p = exp(s[j] - mx);
        den += p;
        const uint16_t* vr = v + kvh * sv0 + j * sv1;
        for (int c = 0; c < D; ++c) o[c] += p * (double)elem(vr[c]);
      }
      for (int c = 0; c < D; ++c) o[c] /= den;
      if (key_mask && !key_mask[b * smb + qabs])
        for (int c = 0; c < D; ++c) o[c] = 0.0;
    }
    free(s);
    free(use);
  }
  return err;
}

/* Per-row symmetric int8 (modal_rd/kv_int8.py:19-22): x is bf16 (kind 0), fp32 (kind 1) or fp16 (kind 2) rows of
 * length d with row stride sx; 16-bit elements are exact in fp32. */
static float orc_elem(const void* x, int kind, int64_t i) {
  if (kind == 1) return ((const float*)x)[i];
  const uint16_t h = ((const uint16_t*)x)[i];
  return kind == 2 ? f16_to_f32(h) : bf16_to_f32(h);
}

int orc_quantize(const void* x, int in_kind, int64_t sx, int64_t rows, int d, float min_scale, int8_t* qo,
                 float* scale_f32, uint16_t* scale_f16) {
  for (int64_t r = 0; r < rows; ++r) {
    float amax = 0.0f;
    for (int c = 0; c < d; ++c) {
      float xv = orc_elem(x, in_kind, r * sx + c);
      float a = fabsf(xv);
      if (a > amax) amax = a;
    }
    float sc = amax / 127.0f;
    if (sc < min_scale) sc = min_scale;
    for (int c = 0; c < d; ++c) {
      float xv = orc_elem(x, in_kind, r * sx + c);
      float qv = nearbyintf(xv / sc);
      if (qv > 127.0f) qv = 127.0f;
      if (qv < -127.0f) qv = -127.0f;
      qo[r * d + c] = (int8_t)qv;
    }
    if (scale_f32) scale_f32[r] = sc;
    if (scale_f16) {
      scale_f16[r] = f32_to_f16_rne(sc);
    }
  }
  return 0;
}

/* Dequantise with an fp16 (scale_is_f16) or fp32 scale; writes fp32. */
int orc_dequantize(const int8_t* qv, const void* scale, int scale_is_f16, int64_t rows, int d, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    float sc;
    if (scale_is_f16) {
      sc = f16_to_f32(((const uint16_t*)scale)[r]);
    } else {
      sc = ((const float*)scale)[r];
    }
    for (int c = 0; c < d; ++c) out[r * d + c] = (float)qv[r * d + c] * sc;
  }
  return 0;
}

/*
 * Exact (dense) attention of one decode token over n cached rows of a token-major int8 cache.
 *   q [H, D] bf16; k8/v8 [cap, Hkv, D] int8; ks/vs [cap, Hkv] scales (fp16 or fp32); out [H, D] float64.
 */
int orc_decode(const uint16_t* q, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
               int scale_is_f16, int n, int H, int Hkv, int D, double scale, double* out) {
  if (H % Hkv) return -1;
  int G = H / Hkv;
  double* s = (double*)malloc(sizeof(double) * (size_t)n);
  if (!s) return -3;
  for (int h = 0; h < H; ++h) {
    int g = h / G;
    double mx = -INFINITY;
    for (int j = 0; j < n; ++j) {
      float sk;
      if (scale_is_f16) sk = f16_to_f32(((const uint16_t*)ks)[(int64_t)j * Hkv + g]);
      else sk = ((const float*)ks)[(int64_t)j * Hkv + g];
      const int8_t* kr = k8 + ((int64_t)j * Hkv + g) * D;
      double acc = 0;
      for (int c = 0; c < D; ++c) acc += (double)bf16_to_f32(q[h * D + c]) * (double)((float)kr[c] * sk);
      s[j] = acc * scale;
      if (s[j] > mx) mx = s[j];
    }
    double den = 0;
    double* o = out + (size_t)h * D;
    for (int c = 0; c < D; ++c) o[c] = 0;
    for (int j = 0; j < n; ++j) {
      float sv;
      if (scale_is_f16) sv = f16_to_f32(((const uint16_t*)vs)[(int64_t)j * Hkv + g]);
      else sv = ((const float*)vs)[(int64_t)j * Hkv + g];
      double p = exp(s[j] - mx);
      den += p;
      const int8_t* vr = v8 + ((int64_t)j * Hkv + g) * D;
      for (int c = 0; c < D; ++c) o[c] += p * (double)((float)vr[c] * sv);
    }
    for (int c = 0; c < D; ++c) o[c] /= den;
  }
  free(s);
  return 0;
}
