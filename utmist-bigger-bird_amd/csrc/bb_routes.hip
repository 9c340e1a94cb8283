// Routing for Bigger Bird v3 prefill (modal_rd/attention.py:143-174 of the reference): for every query head, the
// mean (or max) softmax probability that its r route queries give to each key, then the `budget` best keys in
// [sink, n - window), returned ascending as int32.
//
// The arithmetic is fixed so that results are reproducible bit for bit on any device and by the CPU oracle:
//   s    = bf16_rne(q.k in the reference's order)   torch's CPU bf16 matmul (oneDNN, AMX-BF16): per 32-element block
//                                                   of d, fp32 chains over the even and the odd elements, then
//                                                   acc = acc + (even + odd); one RNE step to bf16
//          fp16_rne(q.k, one sequential fp32 chain) fp16 q and k: torch's CPU fp16 matmul; the workspace then holds
//                                                   fp16 scores
//   x    = fp32(s * scaling); M = row max over causal keys j <= qpos
//   e    = det_exp2(fp32(fp32(x - M) * log2e))
//   Z    = sum floor(e * 2^40) (uint64)    p = fp32(e * fp32(2^40 / double(Z)))
//   P_j  = sum_i floor(p_ij * 2^40)  (or max_i for max pooling); top-budget by (P desc, index asc).
// Integer sums make every reduction order-independent; there are no floating-point atomics.
//
// Kernels (all on the caller's stream, no host synchronisation):
//   scores_kernel   scores of G*r route rows against a 256-key range, bf16 to the workspace, partial row max
//   rowmax_kernel   partial maxima -> row max
//   rowsum_kernel   fixed-point partial row sums over 1024-key blocks
//   invz_kernel     partial sums -> fp32 scale 2^40 / Z per row
//   pooled_kernel   per (head, key): pooled fixed-point probability over the r rows
//   topk_*_kernel   top-budget per head: log-linear histogram over many workgroups, the threshold bin, compaction of
//                   the keys above it and of its candidates, exact choice among the candidates (value desc, index asc)
//                   and ascending emission through a bitmap; an MSD radix select over the whole range when the
//                   candidates overflow (heavy ties)
#include <string.h>

#include "bb_common.h"
#include "bb_internal.h"
#include "bb_topk.h"

// Every rounding step above is part of the contract: no fused multiply-add contraction in this file.
#pragma clang fp contract(off)

namespace bb {
namespace {

constexpr int kScoreKeys = 32;    // keys per scores_kernel block (8 key groups of 4)
constexpr int kScoreIters = 16;   // fewest key blocks per scores workgroup (RouteGeom::iters: 16, 32, 64 or 128)
constexpr int kSumKeys = 1024;    // keys per rowsum_kernel workgroup
constexpr int kPoolKeys = 512;    // keys per pooled_kernel workgroup (2 per thread)
constexpr int kMaxRows = 256;     // route rows (G * r) per scores_kernel workgroup (more rows use more row blocks)
constexpr float kFixOne = 1099511627776.0f;  // 2^40

BB_DEV uint64_t fix40(float v) { return (uint64_t)(v * kFixOne); }

// A stored score (bf16 bits, or fp16 bits for fp16 inputs) as fp32; -inf marks a masked key in either type.
template <bool F16>
BB_DEV float score_f32(uint16_t s) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, s);
  else return bf16_to_f32(s);
}
template <bool F16>
BB_DEV uint16_t score_bits(float x) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)x);  // round to nearest even
  else return f32_to_bf16(x);
}
template <bool F16>
constexpr uint16_t kScoreNegInf = F16 ? 0xfc00u : 0xff80u;

struct RouteGeom {
  int G, rows, n_kb1, n_kb2, row_blocks;
  int iters;  // key blocks of kScoreKeys per scores workgroup: n_kb1 = ceil(n / (kScoreKeys iters))
  int sum_rows, sum_splits;  // rowsum_kernel: rows per workgroup (a multiple of 4) and row slices
  int64_t ns;  // score row stride: n rounded up to 8 (16-byte aligned rows)
};

// Scores: one workgroup = up to 256 route rows of one KV head x g.iters blocks of kScoreKeys keys.
// Q^T stays in LDS for the whole key range; each key block is staged as fp32 K^T. Thread t owns rows
// 8*(t%32)..+7 and keys 4*(t/32)..+3 of a block. Every score is built in the reference's accumulation order: per
// 32-element block of d, two sequential fp32 chains over the even and the odd elements (fmaf of two bf16 values is
// one rounding of the exact product sum), then acc = acc + (even + odd); for fp16 inputs (F16) one sequential chain
// over d (an fp16 product is exact in fp32 as well) and the result rounded to fp16.
// LDS of scores_kernel. bf16: K^T staged in fp32 (the chains take fp32 operands). fp16: K^T kept in fp16 (the FMAs take
// fp16 operands directly) and the row-max partials share its space after the last block, so that two workgroups fit
// a CU (74 KB each at head_dim 128).
template <int D, bool F16>
struct ScoresSmem {
  uint16_t qs[D][kMaxRows];                              // Q^T (16-bit)
  float ks[D][kScoreKeys + 4];                           // K^T (fp32), padded rows
  float rmax_part[kMaxRows][kScoreKeys / 4 + 1];
};
template <int D>
struct ScoresSmem<D, true> {
  uint16_t qs[D][kMaxRows];
  union {
    uint16_t ks[D][kScoreKeys + 8];                      // K^T (fp16), padded rows
    float rmax_part[kMaxRows][kScoreKeys / 4 + 1];       // after the last block
  };
};

template <int D, bool F16>
__global__ __launch_bounds__(256) void scores_kernel(RoutesParams p, RouteGeom g, float* __restrict__ pmax) {
  static_assert(D % 32 == 0, "head_dim must be a multiple of 32");
  __shared__ __attribute__((aligned(16))) ScoresSmem<D, F16> sm;
  auto& qs = sm.qs;
  auto& ks = sm.ks;
  auto& rmax_part = sm.rmax_part;
  const int tid = threadIdx.x;
  const int kchunk = blockIdx.x, rblk = blockIdx.y, bkv = blockIdx.z;
  const int batch = bkv / p.Hkv, kvh = bkv % p.Hkv;
  const int row0 = rblk * kMaxRows;
  const int nrows = g.rows - row0 < kMaxRows ? g.rows - row0 : kMaxRows;

  // stage Q^T: row -> (head slot, query i)
  for (int e = tid; e < kMaxRows * (D / 8); e += 256) {
    const int row = e / (D / 8), c8 = e % (D / 8);
    u32x4_t v = {0, 0, 0, 0};
    if (row < nrows) {
      const int rr = row0 + row, hs = rr / p.r, i = rr % p.r;
      const int head = batch * p.H + kvh * g.G + hs;
      v = ld16(p.q + (int64_t)head * p.sq0 + p.qpos[i] * p.sq1 + 8 * c8);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      qs[8 * c8 + 2 * w][row] = (uint16_t)(v[w] & 0xffffu);
      qs[8 * c8 + 2 * w + 1][row] = (uint16_t)(v[w] >> 16);
    }
  }

  const int rg = tid & 31, kg = tid >> 5;
  int64_t qp[8];
#pragma unroll
  for (int a = 0; a < 8; ++a) {
    const int row = 8 * rg + a;
    qp[a] = row < nrows ? p.qpos[(row0 + row) % p.r] : -1;
  }
  float rmax[8];
#pragma unroll
  for (int a = 0; a < 8; ++a) rmax[a] = -__builtin_huge_valf();
  const uint16_t* kbase = p.k + (int64_t)bkv * p.sk0;
  uint16_t* srow_base = p.scores + (int64_t)bkv * g.rows * g.ns;

  // K blocks: thread t holds the 16-byte units t, t + 256, ... of a block; the next block's loads are in flight
  // while the current one is scored
  constexpr int KPT = (kScoreKeys * (D / 8) + 255) / 256;
  auto kload = [&](int it, u32x4_t (&dst)[KPT]) {
    const int64_t jb = ((int64_t)kchunk * g.iters + it) * kScoreKeys;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = tid + 256 * u;
      const int64_t j = jb + e / (D / 8);
      dst[u] = e < kScoreKeys * (D / 8) && j < p.n ? ld16(kbase + j * p.sk1 + 8 * (e % (D / 8))) : u32x4_t{0, 0, 0, 0};
    }
  };
  u32x4_t knext[KPT];
  kload(0, knext);

  for (int it = 0; it < g.iters; ++it) {
    const int64_t j0 = ((int64_t)kchunk * g.iters + it) * kScoreKeys;
    if (j0 >= p.n) break;
    __syncthreads();  // previous block's K^T fully consumed (and Q^T staged on the first pass)
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = tid + 256 * u;
      if (e < kScoreKeys * (D / 8)) {
        const int key = e / (D / 8), c8 = e % (D / 8);
        const u32x4_t v = knext[u];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (F16) {
            ks[8 * c8 + 2 * w][key] = (uint16_t)(v[w] & 0xffffu);
            ks[8 * c8 + 2 * w + 1][key] = (uint16_t)(v[w] >> 16);
          } else {
            ks[8 * c8 + 2 * w][key] = bf16_to_f32((uint16_t)(v[w] & 0xffffu));
            ks[8 * c8 + 2 * w + 1][key] = bf16_to_f32((uint16_t)(v[w] >> 16));
          }
        }
      }
    }
    __syncthreads();
    if (it + 1 < g.iters) kload(it + 1, knext);

    float acc[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
    if constexpr (F16) {
#pragma unroll 2
      for (int dd = 0; dd < D; ++dd) {
        const u32x4_t qv = *reinterpret_cast<const u32x4_t*>(&qs[dd][8 * rg]);
        const u32x2_t kv = *reinterpret_cast<const u32x2_t*>(&ks[dd][4 * kg]);
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          const float fq = score_f32<true>((uint16_t)(qv[a >> 1] >> (16 * (a & 1))));
#pragma unroll
          for (int b = 0; b < 4; ++b)
            acc[a][b] = __builtin_fmaf(fq, score_f32<true>((uint16_t)(kv[b >> 1] >> (16 * (b & 1)))), acc[a][b]);
        }
      }
    }
    for (int d0 = 0; !F16 && d0 < D; d0 += 32) {
      float ev[8][4], od[8][4];
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) ev[a][b] = od[a][b] = 0.0f;
#pragma unroll 4
      for (int t = 0; t < 16; ++t) {
        const int de = d0 + 2 * t;
        const u32x4_t qe = *reinterpret_cast<const u32x4_t*>(&qs[de][8 * rg]);
        const u32x4_t qo = *reinterpret_cast<const u32x4_t*>(&qs[de + 1][8 * rg]);
        const f32x4_t ke = *reinterpret_cast<const f32x4_t*>(&ks[de][4 * kg]);
        const f32x4_t ko = *reinterpret_cast<const f32x4_t*>(&ks[de + 1][4 * kg]);
#pragma unroll
        for (int a = 0; a < 8; ++a) {
          const float fe = bf16_to_f32((uint16_t)(qe[a >> 1] >> (16 * (a & 1))));
          const float fo = bf16_to_f32((uint16_t)(qo[a >> 1] >> (16 * (a & 1))));
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            ev[a][b] = __builtin_fmaf(fe, ke[b], ev[a][b]);
            od[a][b] = __builtin_fmaf(fo, ko[b], od[a][b]);
          }
        }
      }
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = acc[a][b] + (ev[a][b] + od[a][b]);
    }

    // round to bf16, causal mask, store, running row max of x = s * scaling
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      const int row = 8 * rg + a;
      const int64_t jj = j0 + 4 * kg;
      uint16_t sb[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t j = jj + b;
        sb[b] = kScoreNegInf<F16>;
        if (j < p.n && j <= qp[a]) {
          sb[b] = score_bits<F16>(acc[a][b]);
          rmax[a] = fmaxf(rmax[a], score_f32<F16>(sb[b]) * p.scaling);
        }
      }
      if (row < nrows) {
        uint16_t* dst = srow_base + (int64_t)(row0 + row) * g.ns + jj;
        if (jj + 4 <= p.n) {
          *reinterpret_cast<u32x2_t*>(dst) =
              u32x2_t{(uint32_t)sb[0] | ((uint32_t)sb[1] << 16), (uint32_t)sb[2] | ((uint32_t)sb[3] << 16)};
        } else {
          for (int b = 0; b < 4 && jj + b < p.n; ++b) dst[b] = sb[b];
        }
      }
    }
  }
  if constexpr (F16) __syncthreads();  // rmax_part shares the K^T space
#pragma unroll
  for (int a = 0; a < 8; ++a) rmax_part[8 * rg + a][kg] = rmax[a];
  __syncthreads();
  if (tid < nrows) {
    float mx = rmax_part[tid][0];
#pragma unroll
    for (int b = 1; b < kScoreKeys / 4; ++b) mx = fmaxf(mx, rmax_part[tid][b]);
    pmax[((int64_t)bkv * g.n_kb1 + kchunk) * g.rows + row0 + tid] = mx;
  }
}

// MFMA scores with exact fix-up (head_dim 128). The bf16 score of every (route row, key) must be the one the
// reference order above produces. Both that order and the MFMA path sum the same 128 exact bf16 products
// p_d = q_d k_d in fp32, and each result's distance from the exact sum is bounded per product (u = 2^-24; every
// rounding of a partial sum x errs by at most u |x|, and |x| <= the sum of |p_d| over the products in it):
//   * reference order, d = 32 c + 2 t + parity: the even / odd chain of block c rounds at its steps t' = 1..15 (step 0
//     adds to zero exactly), then once for even + odd, then at the block sums c' = 1..3. Product d passes through
//     (16 - max(t, 1)) + 1 + (4 - max(c, 1)) roundings (19 at most, 11.7 on average against the 21 of a uniform
//     bound).
//   * MFMA path: slice s (d = 16 s .. 16 s + 15) is one MFMA with a zero accumulator, its 16 products aligned to the
//     largest one and truncated below 2^-23 of it (the error model measured on the hardware), then rounded: at most
//     32 u M_s + 2 u sum_s|p|, with M_s = max over the slice of |p_d| <= max|q_d| max|k_d|; the eight slice partials
//     are then added in order, so slice s passes through 8 - max(s, 1) more roundings.
// So |reference - MFMA| <= u (sum_d c_d |q_d| |k_d| + 32 sum_s max_s|q| max_s|k|) with
// c_d = (16 - max(t, 1)) + 1 + (4 - max(c, 1)) + (10 - max(s, 1)). One accumulating MFMA chain computes that bound
// per score: |K| against the weighted row c_d |q_d| (rounded up to bf16), then one more MFMA of the per-slice maxima
// of |K| against 32 x the per-slice maxima of |Q|. The bound's own MFMA rounding (all terms are non-negative; below
// 2^-16 relative), the fp32 evaluation of the bound and second-order terms are covered by the factor 1 + 2^-10 in
// kScoreSlack, underflow by the absolute 2^-100. If s - B and s + B round to the same bf16 value, so does the
// reference-order score (it is an fp32 value in [s - B, s + B]), and that value is taken; otherwise (a score near a
// rounding boundary, or tiny) the score is recomputed in the reference order.
//
// Workgroup: one KV head, up to 256 route rows (G r), g.iters blocks of 32 keys; 8 waves, wave w owns rows
// 32w..32w+31 (one MFMA block, Q^T operands in registers; two waves per SIMD hide each other's MFMA and LDS
// latencies). Per key block S^T = K Q^T (eight slice partials) and the bound run on 17 MFMAs with K from LDS. The
// flagged scores of all eight waves go to one workgroup list, which every thread then works through (about 2% of
// the scores: a few wave-iterations per block for the whole workgroup, instead of one per wave). Scores go through an
// LDS tile per wave so that fix-ups land before one coalesced store, made at the start of the next block.
constexpr float kScoreSlack = 5.9662e-8f;  // u (1 + 2^-10)
constexpr int kMsRowPitch = 136;           // bf16 elements per staged Q row (272 bytes: conflict-free row reads)
constexpr int kMsTilePitch = 40;           // bf16 per score-tile row (80 bytes: conflict-free 8-byte row writes)

// Weight c_d of the certification bound for element d of a 128-element dot product (see above).
BB_DEV int bound_weight(int d) {
  const int c = d >> 5, t = (d & 31) >> 1, s = d >> 4;
  return (16 - (t > 1 ? t : 1)) + 1 + (4 - (c > 1 ? c : 1)) + (10 - (s > 1 ? s : 1));
}

// Magnitude maximum of the eight bf16 values of a fragment (abs bit patterns order as unsigned integers).
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
BB_DEV uint32_t abs_max8(u32x4_t a) {
  const u16x2_t m = __builtin_elementwise_max(
      __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a[0]), __builtin_bit_cast(u16x2_t, a[1])),
      __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a[2]), __builtin_bit_cast(u16x2_t, a[3])));
  return m[0] > m[1] ? m[0] : m[1];
}

// NW waves of 32 route rows each (NW = 8: 256 rows of one KV head; groups of 1 or 2 query heads have only 64 or 128
// rows, so their workgroups are 2 or 4 waves and no wave computes rows that do not exist)
template <int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void scores_mfma_kernel(RoutesParams p, RouteGeom g, float* __restrict__ pmax) {
  static_assert(D == 128, "MFMA scores are built for head_dim 128");
  static_assert(NW == 2 || NW == 4 || NW == 8, "K staging splits 512 16-byte pieces evenly over the threads");
  constexpr int ROWS = 32 * NW, NT = 64 * NW, KPT = kScoreKeys * (D / 8) / NT;  // K pieces per thread
  __shared__ __attribute__((aligned(16))) uint16_t qs[ROWS][kMsRowPitch];   // Q rows (bf16)
  __shared__ __attribute__((aligned(16))) uint16_t kt[kScoreKeys][D];       // K block, chunk c of key j at c ^ (j % 16)
  __shared__ __attribute__((aligned(16))) float kf[kScoreKeys][D];          // the same block in fp32 (same slots)
  __shared__ __attribute__((aligned(16))) uint16_t st[NW][32][kMsTilePitch];  // per-wave score tile (bf16)
  __shared__ uint16_t flist[NW * 32 * kScoreKeys];                          // fix-ups: wave << 10 | lane << 4 | r
  __shared__ uint32_t fcount;                                               // entries of flist
  __shared__ uint32_t rmax_fix[ROWS];                                       // ordered-float max of fixed-up x
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31, h = lane >> 5;
  const int kchunk = blockIdx.x, rblk = blockIdx.y, bkv = blockIdx.z;
  const int batch = bkv / p.Hkv, kvh = bkv % p.Hkv;
  const int row0 = rblk * ROWS;
  const int nrows = g.rows - row0 < ROWS ? g.rows - row0 : ROWS;

  // stage Q rows: row -> (head slot, route query i)
  for (int e = tid; e < ROWS * (D / 8); e += NT) {
    const int row = e / (D / 8), c8 = e % (D / 8);
    u32x4_t v = {0, 0, 0, 0};
    if (row < nrows) {
      const int rr = row0 + row, hs = rr / p.r, i = rr % p.r;
      const int head = batch * p.H + kvh * g.G + hs;
      v = ld16(p.q + (int64_t)head * p.sq0 + p.qpos[i] * p.sq1 + 8 * c8);
    }
    *reinterpret_cast<u32x4_t*>(&qs[row][8 * c8]) = v;
  }
  for (int e = tid; e < ROWS; e += NT) rmax_fix[e] = 0u;  // ordered key below every float
  if (tid == 0) fcount = 0u;
  __syncthreads();

  // B operands (Q^T of row 32 wave + li) and the causal limit
  const int myrow = 32 * wave + li;
  constexpr u32x4_t kAbs = {0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu};
  u32x4_t qf[D / 16];
#pragma unroll
  for (int dk = 0; dk < D / 16; ++dk) qf[dk] = *reinterpret_cast<const u32x4_t*>(&qs[myrow][16 * dk + 8 * h]);
  // bound operands: c_d |q_d| rounded up to bf16 (this lane holds d = 16 dk + 8 h + e), and 32 x the per-slice
  // maxima of |q| (positions 0..7 of the lane with h = 0, zeros at positions 8..15)
  u32x4_t qw[D / 16];
  u32x4_t mq32 = {0, 0, 0, 0};
#pragma unroll
  for (int dk = 0; dk < D / 16; ++dk) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t packed = 0;
#pragma unroll
      for (int hw = 0; hw < 2; ++hw) {
        const float a = __uint_as_float(((qf[dk][w] >> (16 * hw)) & 0x7fffu) << 16);
        const float v = a * (float)bound_weight(16 * dk + 8 * h + 2 * w + hw);  // exact: <= 13 significant bits
        packed |= ((__float_as_uint(v) + 0xffffu) >> 16) << (16 * hw);          // rounded up to bf16
      }
      qw[dk][w] = packed;
    }
    const uint32_t half = abs_max8(qf[dk] & u32x4_t{0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu, 0x7fff7fffu});
    const auto sw = __builtin_amdgcn_permlane32_swap(half, half, false, false);
    const uint32_t mq = sw[0] > sw[1] ? sw[0] : sw[1];                 // max |q| over slice dk of row li
    const uint32_t m32 = __float_as_uint(__uint_as_float(mq << 16) * 32.0f) >> 16;  // exact
    if (h == 0) mq32[dk >> 1] |= m32 << (16 * (dk & 1));
  }
  const int64_t qlim = myrow < nrows ? p.qpos[(row0 + myrow) % p.r] : -1;
  float rmax = -__builtin_huge_valf();
  const uint16_t* kbase = p.k + (int64_t)bkv * p.sk0;
  uint16_t* srow_base = p.scores + (int64_t)bkv * g.rows * g.ns;
  uint16_t (*tile)[kMsTilePitch] = st[wave];
  // tile -> scores for the block at key jb: 32 rows x 32 keys, one 16-byte chunk (8 keys) per lane and step
  auto store_tile = [&](int64_t jb) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int e = 64 * s2 + lane, lrow = e >> 2, c = e & 3;
      const int row = 32 * wave + lrow;
      const int64_t j = jb + 8 * c;
      if (row < nrows && j + 8 <= g.ns)
        st16(srow_base + (int64_t)(row0 + row) * g.ns + j, *reinterpret_cast<const u32x4_t*>(&tile[lrow][8 * c]));
    }
  };

  // K blocks: piece e = tid + NT x (key e / 16, chunk e % 16) is 16 bytes; the next block's load is in flight while
  // the current one is processed
  auto kload = [&](int it, u32x4_t (&dst)[KPT]) {
#pragma unroll
    for (int x = 0; x < KPT; ++x) {
      const int e = tid + NT * x;
      const int64_t j = ((int64_t)kchunk * g.iters + it) * kScoreKeys + (e >> 4);
      dst[x] = j < p.n ? ld16(kbase + j * p.sk1 + 8 * (e & 15)) : u32x4_t{0, 0, 0, 0};
    }
  };
  u32x4_t knext[KPT];
  kload(0, knext);
  int64_t jlast = -1;  // key of the block whose tile is still to be stored
  for (int it = 0; it < g.iters; ++it) {
    const int64_t j0 = ((int64_t)kchunk * g.iters + it) * kScoreKeys;
    if (j0 >= p.n) break;
    __syncthreads();  // the previous block's K and fix-up list are no longer read, and its fix-ups have landed
    if (jlast >= 0) store_tile(jlast);
    jlast = j0;
    if (tid == 0) fcount = 0u;
#pragma unroll
    for (int x = 0; x < KPT; ++x) {  // stage the K block: bf16 for the MFMA fragments, fp32 for the fix-ups
      const int e = tid + NT * x, skey = e >> 4, schunk = e & 15;
      const int slot = 8 * (schunk ^ (skey & 15));  // chunk c of key j in slot c ^ (j % 16)
      const u32x4_t v = knext[x];
      *reinterpret_cast<u32x4_t*>(&kt[skey][slot]) = v;
      *reinterpret_cast<f32x4_t*>(&kf[skey][slot]) = f32x4_t{
          __uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xffff0000u), __uint_as_float(v[1] << 16),
          __uint_as_float(v[1] & 0xffff0000u)};
      *reinterpret_cast<f32x4_t*>(&kf[skey][slot + 4]) = f32x4_t{
          __uint_as_float(v[2] << 16), __uint_as_float(v[2] & 0xffff0000u), __uint_as_float(v[3] << 16),
          __uint_as_float(v[3] & 0xffff0000u)};
    }
    __syncthreads();
    if (it + 1 < g.iters) kload(it + 1, knext);

    // S^T = K Q^T as eight slice partials (zero accumulators) summed in fp32, and the bound's sum of c_d |q_d| |k_d|
    // (each partial is added one step later, while the next slice's MFMAs run: two partials live at a time)
    f32x16_t acc = f32x16_t{}, aac = f32x16_t{}, prev = f32x16_t{};
    uint32_t mk[D / 16];  // max |k| over this lane's half of slice dk (key li)
#pragma unroll
    for (int dk = 0; dk < D / 16; ++dk) {
      const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(&kt[li][8 * ((2 * dk + h) ^ (li & 15))]);
      const f32x16_t cur = mfma32(as_bf16x8(kv), as_bf16x8(qf[dk]), f32x16_t{});
      const u32x4_t ka = kv & kAbs;
      aac = mfma32(as_bf16x8(ka), as_bf16x8(qw[dk]), aac);
      mk[dk] = abs_max8(ka);
      if (dk == 1) acc = prev;
      else if (dk > 1) acc = acc + prev;
      prev = cur;
      __builtin_amdgcn_sched_barrier(0);
    }
    acc = acc + prev;
    {  // + 32 sum_s max_s|k| max_s|q|: slice maxima of key li (both halves) at positions 0..7 of the h = 0 lane
      u32x4_t mka = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = mk[2 * i] | (mk[2 * i + 1] << 16);
        const auto sw = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        const u16x2_t m = __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, sw[0]), __builtin_bit_cast(u16x2_t, sw[1]));
        mka[i] = h == 0 ? __builtin_bit_cast(uint32_t, m) : 0u;
      }
      aac = mfma32(as_bf16x8(mka), as_bf16x8(mq32), aac);
    }

    // certify or flag every score; lane (li, h) holds row li's keys 8 (r / 4) + 4 h + r % 4 of the block
    int64_t lim64 = (qlim < p.n - 1 ? qlim : p.n - 1) - j0;  // live keys: kk <= lim
    const int lim = lim64 < -1 ? -1 : (lim64 > kScoreKeys ? kScoreKeys : (int)lim64);
    const int limh = lim - 4 * h;  // compared with the lane-independent part of kk
    uint32_t fixbits = 0;  // bit r: score r of this lane needs the fix-up
    uint32_t outw[8];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = 8 * (r >> 2) + 4 * h + (r & 3);
      const float sv = acc[r];
      const float bound = kScoreSlack * aac[r] + 7.9e-31f;
      const uint32_t pr = pack_bf16x2(sv - bound, sv + bound);
      const bool live = 8 * (r >> 2) + (r & 3) <= limh;
      const bool sure = (pr & 0xffffu) == (pr >> 16);
      uint32_t out = 0xff80u;  // -inf for masked keys
      if (live && sure) {
        out = pr & 0xffffu;
        rmax = fmaxf(rmax, __uint_as_float(out << 16) * p.scaling);
      }
      if (r & 1) outw[r >> 1] |= out << 16;
      else outw[r >> 1] = out;
      if ((r & 3) == 3)  // keys 8 (r / 4) + 4 h + 0..3 are consecutive: one 8-byte store
        *reinterpret_cast<u32x2_t*>(&tile[li][kk - 3]) = u32x2_t{outw[(r >> 1) - 1], outw[r >> 1]};
      fixbits |= (uint32_t)(live && !sure) << r;
    }
    // this wave's flagged scores go to the workgroup list: one atomic per wave reserves their slots
    {
      const uint32_t cnt = __builtin_popcount(fixbits);
      uint32_t incl = cnt;  // inclusive prefix sum over the wave's lanes
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off);
        if (lane >= off) incl += t;
      }
      const uint32_t total = __shfl(incl, 63);
      uint32_t base = 0;
      if (lane == 0 && total) base = atomicAdd(&fcount, total);
      base = __shfl(base, 0) + incl - cnt;
      const uint32_t ebase = ((uint32_t)wave << 10) | ((uint32_t)lane << 4);
      for (uint32_t b = fixbits; b; b &= b - 1) flist[base++] = (uint16_t)(ebase | (uint32_t)__builtin_ctz(b));
    }
    __syncthreads();  // the list is complete

    // exact recomputation of the flagged scores in the reference order, by every thread of the workgroup
    const uint32_t nfix = fcount;
    for (uint32_t e = tid; e < nfix; e += NT) {
      const uint32_t ent = flist[e];
      const int ew = (int)(ent >> 10), el = (int)((ent >> 4) & 63u), er = (int)(ent & 15u);
      const int lrow = el & 31, kk = 8 * (er >> 2) + 4 * (el >> 5) + (er & 3);
      const uint16_t* qr = qs[32 * ew + lrow];
      const float* kr = kf[kk];
      const int ksw = kk & 15;  // chunk c of key kk sits at slot c ^ (kk % 16)
      float accx = 0.0f;
#pragma unroll
      for (int blk = 0; blk < D / 32; ++blk) {
        float ev = 0.0f, od = 0.0f;
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          const int c = 4 * blk + c2;  // 8-element chunk of d
          const u32x4_t qv = *reinterpret_cast<const u32x4_t*>(qr + 8 * c);
          const f32x4_t k0 = *reinterpret_cast<const f32x4_t*>(kr + 8 * (c ^ ksw));
          const f32x4_t k1 = *reinterpret_cast<const f32x4_t*>(kr + 8 * (c ^ ksw) + 4);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float ke = w < 2 ? k0[2 * w] : k1[2 * w - 4], ko = w < 2 ? k0[2 * w + 1] : k1[2 * w - 3];
            ev = __builtin_fmaf(__uint_as_float(qv[w] << 16), ke, ev);
            od = __builtin_fmaf(__uint_as_float(qv[w] & 0xffff0000u), ko, od);
          }
        }
        accx = accx + (ev + od);
      }
      const uint16_t out = f32_to_bf16(accx);
      st[ew][lrow][kk] = out;
      atomicMax(&rmax_fix[32 * ew + lrow], float_to_ordered(bf16_to_f32(out) * p.scaling));
    }
  }
  // the last block's fix-ups, then its tile; row maxima: the two halves of a row's lanes, then the fixed-up scores
  __syncthreads();
  if (jlast >= 0) store_tile(jlast);
  {
    const float mx = xhalf_max(rmax);
    if (h == 0 && myrow < nrows) {
      const uint32_t fk = rmax_fix[myrow];
      const float fx = fk ? ordered_to_float(fk) : -__builtin_huge_valf();
      pmax[((int64_t)bkv * g.n_kb1 + kchunk) * g.rows + row0 + myrow] = fmaxf(mx, fx);
    }
  }
}

// One wave per (KV head, route row): lanes stride over the key-block partials, then a wave maximum.
__global__ __launch_bounds__(64) void rowmax_kernel(RoutesParams p, RouteGeom g, const float* __restrict__ pmax) {
  const int row = blockIdx.x, bkv = blockIdx.y, lane = threadIdx.x;
  float mx = -__builtin_huge_valf();
  for (int kb = lane; kb < g.n_kb1; kb += 64) mx = fmaxf(mx, pmax[((int64_t)bkv * g.n_kb1 + kb) * g.rows + row]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if (lane == 0) p.rowmax[(int64_t)bkv * g.rows + row] = __float_as_uint(mx);
}

// fix40(det_exp2(y) * scale) as an integer-valued float below 2^41, for y <= 0 (or -inf / NaN) and 0 < scale <= 1,
// bit for bit: det_exp2's ldexp and fix40's scale by 2^40 fold into one exact ldexp of fl(p scale) (det_exp2(y) scale
// rounds to fl(p scale) 2^n whenever that is a normal float; otherwise both results truncate to 0), and fix40's
// floor is one truncation. y <= -100 and NaN give 0 as in det_exp2: clamped to -101, the value stays below 2^-59.
BB_DEV float fix40_exp2(float y, float scale) {
  y = fmaxf(y, -101.0f);
  const float n = rintf(y);
  const float f = y - n;
  float q = 1.5252733804059840e-05f;
  q = fmaf(q, f, 1.5403530393381610e-04f);
  q = fmaf(q, f, 1.3333558146428443e-03f);
  q = fmaf(q, f, 9.6181291076284772e-03f);
  q = fmaf(q, f, 5.5504108664821580e-02f);
  q = fmaf(q, f, 2.4022650695910071e-01f);
  q = fmaf(q, f, 6.9314718055994531e-01f);
  q = fmaf(q, f, 1.0f);
  return truncf(ldexpf(q * scale, (int)(n + 40.0f)));
}

// Fixed-point partial row sums: one wave per row (4 rows in flight per workgroup), 16 keys per lane. The rows of a
// key block may be cut into blockIdx.z slices of g.sum_rows rows, so short sequences still fill the chip. The terms
// are integers below 2^41, so their sums stay exact in double precision (1024 terms per workgroup row < 2^51).
template <bool F16>
__global__ __launch_bounds__(256) void rowsum_kernel(RoutesParams p, RouteGeom g, uint64_t* __restrict__ psum) {
  const int kb = blockIdx.x, bkv = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r_begin = blockIdx.z * g.sum_rows;
  const int r_end = r_begin + g.sum_rows < g.rows ? r_begin + g.sum_rows : g.rows;
  const int64_t j0 = (int64_t)kb * kSumKeys + 16 * lane;
  // the next row's scores are loaded while this row's are summed
  u32x4_t na = {0, 0, 0, 0}, nb = {0, 0, 0, 0};
  if (r_begin + wave < r_end && j0 + 16 <= p.n) {
    const uint16_t* src = p.scores + ((int64_t)bkv * g.rows + r_begin + wave) * g.ns + j0;
    na = ld16(src);
    nb = ld16(src + 8);
  }
  for (int row = r_begin + wave; row < r_end; row += 4) {
    const float M = __uint_as_float(p.rowmax[(int64_t)bkv * g.rows + row]);
    const uint16_t* src = p.scores + ((int64_t)bkv * g.rows + row) * g.ns + j0;
    double acc = 0.0;
    if (j0 + 16 <= p.n) {
      const u32x4_t a = na, b = nb;
      if (row + 4 < r_end) {
        na = ld16(src + 4 * g.ns);
        nb = ld16(src + 4 * g.ns + 8);
      }
      uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint16_t sb = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        const float x = score_f32<F16>(sb) * p.scaling;
        acc += (double)fix40_exp2((x - M) * kLog2e, 1.0f);
      }
    } else {
      for (int e = 0; e < 16 && j0 + e < p.n; ++e) {
        const float x = score_f32<F16>(src[e]) * p.scaling;
        acc += (double)fix40_exp2((x - M) * kLog2e, 1.0f);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) psum[((int64_t)bkv * g.n_kb2 + kb) * g.rows + row] = (uint64_t)acc;
  }
}

// One wave per (KV head, route row): integer partial sums (order-free), then 2^40 / Z. The workgroups of the first G
// rows of each KV head also clear that query head's top-k histogram and list counters, which the top-k kernels
// accumulate into.
__global__ __launch_bounds__(64) void invz_kernel(RoutesParams p, RouteGeom g, const uint64_t* __restrict__ psum,
                                                 float* __restrict__ invz, uint32_t* __restrict__ top_hist,
                                                 uint32_t* __restrict__ top_meta) {
  const int row = blockIdx.x, bkv = blockIdx.y, lane = threadIdx.x;
  if (row < g.G) {
    const int head = (bkv / p.Hkv) * p.H + (bkv % p.Hkv) * g.G + row;
    for (int b = lane; b < kTopBins; b += 64) top_hist[(int64_t)head * kTopBins + b] = 0u;
    if (lane < kTopMetaWords) top_meta[kTopMetaWords * head + lane] = 0u;
  }
  uint64_t z = 0;
  for (int kb = lane; kb < g.n_kb2; kb += 64) z += psum[((int64_t)bkv * g.n_kb2 + kb) * g.rows + row];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off);
  if (lane == 0) {
    const int64_t t = (int64_t)bkv * g.rows + row;
    p.rowsum[t] = z;
    invz[t] = (float)(1099511627776.0 / (double)z);
  }
}

// Pooled fixed-point probability per (query head, key): two consecutive keys per thread (one 4-byte score load per
// route row, eight rows' loads in flight), the head's r rows in a loop, sums exact in double precision (64 rows x
// 2^41 < 2^53).
template <bool F16>
__global__ __launch_bounds__(256) void pooled_kernel(RoutesParams p, RouteGeom g, const float* __restrict__ invz) {
  const int64_t j0 = 2 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
  const int head = blockIdx.y;  // over B * H
  if (j0 >= p.n) return;
  const int batch = head / p.H, hh = head % p.H;
  const int kvh = hh / g.G, hs = hh % g.G;
  const int64_t bkv = (int64_t)batch * p.Hkv + kvh;
  const int64_t lo = p.sink, hi = p.n - p.window;  // eligible keys [lo, hi)
  double P0 = 0.0, P1 = 0.0;
  if (j0 + 2 > lo && j0 < hi) {
    // keys past n read as -inf: score rows end at g.ns, a multiple of 8, and the scorer stores -inf there
    const uint16_t* src = p.scores + (bkv * g.rows + (int64_t)hs * p.r) * g.ns + j0;
    const float* mrow = reinterpret_cast<const float*>(p.rowmax) + bkv * g.rows + (int64_t)hs * p.r;
    const float* zrow = invz + bkv * g.rows + (int64_t)hs * p.r;
    int i = 0;
    for (; i < p.r; i += 8) {
      const int nb = p.r - i < 8 ? p.r - i : 8;
      uint32_t w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = u < nb ? *reinterpret_cast<const uint32_t*>(src + (int64_t)(i + u) * g.ns) : 0u;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u >= nb) break;
        const float M = mrow[i + u], iz = zrow[i + u];
        const float x0 = score_f32<F16>((uint16_t)(w[u] & 0xffffu)) * p.scaling;
        const float x1 = score_f32<F16>((uint16_t)(w[u] >> 16)) * p.scaling;
        const double f0 = (double)fix40_exp2((x0 - M) * kLog2e, iz);
        const double f1 = (double)fix40_exp2((x1 - M) * kLog2e, iz);
        if (p.pool_max) {
          P0 = f0 > P0 ? f0 : P0;
          P1 = f1 > P1 ? f1 : P1;
        } else {
          P0 += f0;
          P1 += f1;
        }
      }
    }
  }
  uint64_t* dst = p.pooled + (int64_t)head * p.n + j0;
  dst[0] = j0 >= lo && j0 < hi ? (uint64_t)P0 : 0ull;
  if (j0 + 1 < p.n) dst[1] = j0 + 1 >= lo && j0 + 1 < hi ? (uint64_t)P1 : 0ull;
}

// Eligible range [sink, n - window) of the top-k kernels; n comes from device memory when n_dev is set (decode
// routing on a growing cache), clamped to the row stride.
BB_DEV void top_range(const RoutesParams& p, int64_t& lo, int64_t& cnt) {
  int64_t n = p.n_dev ? *p.n_dev : p.n;
  if (n > p.pstride) n = p.pstride;
  if (n < 0) n = 0;
  lo = p.sink < n ? (p.sink > 0 ? p.sink : 0) : n;
  int64_t hi = n - p.window;
  if (hi > n) hi = n;
  cnt = hi > lo ? hi - lo : 0;
}

// Top-budget selection for one head by one 1024-thread workgroup: MSD radix select over 8-bit digits of the whole
// eligible range, then ordered compaction. The general path (any ties, any budget); topk_final_kernel uses it when
// the candidate set of the fast path overflows.
constexpr int kTopThreads = 1024;

// Inclusive sum over the NT threads of a workgroup in thread order: a shuffle scan per wave, then the wave totals
// through LDS (ws: NT / 64 words). Every thread must call it; `total` receives the workgroup's sum.
template <int NT>
BB_DEV uint32_t block_incl_scan(uint32_t v, uint32_t* ws, uint32_t& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t t = __shfl_up(v, off);
    if (lane >= off) v += t;
  }
  if (lane == 63) ws[wave] = v;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const uint32_t x = ws[w];
    before += w < wave ? x : 0u;
    all += x;
  }
  __syncthreads();  // ws is free again
  total = all;
  return v + before;
}

__device__ __forceinline__ void topk_radix_head(const RoutesParams& p, int head) {
  __shared__ uint32_t hist[256];
  __shared__ uint64_t red[kTopThreads / 64];
  __shared__ uint32_t scan_sel[kTopThreads / 64];
  __shared__ uint64_t s_prefix, s_mask;
  __shared__ int64_t s_need;
  __shared__ int s_exact;

  const int tid = threadIdx.x;
  int64_t lo, cnt;
  top_range(p, lo, cnt);
  const uint64_t* P = p.pooled + (int64_t)head * p.pstride + lo;
  int32_t* out = p.out_idx + (int64_t)head * p.budget;
  for (int i = tid; i < p.budget; i += kTopThreads) out[i] = -1;  // slots past the eligible count read -1
  __syncthreads();
  if (p.budget <= 0 || cnt <= 0) return;

  // global max -> first digit
  uint64_t mx = 0;
  for (int64_t t = tid; t < cnt; t += kTopThreads) mx = P[t] > mx ? P[t] : mx;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint64_t o = __shfl_xor(mx, off);
    mx = o > mx ? o : mx;
  }
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) {
    uint64_t m = 0;
    for (int w = 0; w < kTopThreads / 64; ++w) m = red[w] > m ? red[w] : m;
    red[0] = m;
    s_prefix = 0;
    s_mask = 0;
    s_need = p.budget;
    s_exact = 0;
  }
  __syncthreads();
  const uint64_t gmax = red[0];
  int top_digit = 0;
  if (gmax) top_digit = (63 - __clzll((long long)gmax)) / 8;
  // the most significant digits above top_digit are zero for every value: fixed prefix 0
  uint64_t prefix = 0, mask = top_digit < 7 ? ~((1ull << (8 * (top_digit + 1))) - 1ull) : 0ull;
  if (tid == 0) s_mask = mask;
  __syncthreads();
  for (int digit = top_digit; digit >= 0; --digit) {
    const int shift = 8 * digit;
    for (int b = tid; b < 256; b += kTopThreads) hist[b] = 0;
    __syncthreads();
    prefix = s_prefix;
    mask = s_mask;
    for (int64_t t = tid; t < cnt; t += kTopThreads) {
      const uint64_t v = P[t];
      if ((v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      int64_t need = s_need, cum = 0;
      int bsel = 0;
      for (int b = 255; b >= 0; --b) {
        if (cum + (int64_t)hist[b] >= need) { bsel = b; break; }
        cum += hist[b];
      }
      need -= cum;  // still needed from bin bsel
      s_prefix = prefix | ((uint64_t)bsel << shift);
      s_mask = mask | (255ull << shift);
      s_need = need;
      if ((int64_t)hist[bsel] == need) s_exact = 1;  // whole bin selected: no ties to break
    }
    __syncthreads();
    if (s_exact) break;
  }
  // Final threshold: values matching prefix under mask form the boundary set; `need` of them are taken
  // (all of them when s_exact), lowest indices first.
  prefix = s_prefix;
  mask = s_mask;
  const int64_t need = s_need;
  const int64_t seg = (cnt + kTopThreads - 1) / kTopThreads;
  const int64_t t0 = (int64_t)tid * seg, t1 = t0 + seg < cnt ? t0 + seg : cnt;
  uint32_t nsel = 0, ntie = 0;
  for (int64_t t = t0; t < t1; ++t) {
    const uint64_t v = P[t];
    const uint64_t vm = v & mask;
    if (vm > prefix) ++nsel;
    else if (vm == prefix) ++ntie;
  }
  uint32_t tot;
  const int64_t sel_before = (int64_t)block_incl_scan<kTopThreads>(nsel, scan_sel, tot) - nsel;
  const int64_t tie_before = (int64_t)block_incl_scan<kTopThreads>(ntie, scan_sel, tot) - ntie;
  // position of an element = selected-above before it + ties taken before it
  int64_t taken_ties = tie_before < need ? tie_before : need;
  int64_t pos = sel_before + taken_ties;
  int64_t ties_seen = tie_before;
  for (int64_t t = t0; t < t1; ++t) {
    const uint64_t vm = P[t] & mask;
    bool take = false;
    if (vm > prefix) take = true;
    else if (vm == prefix) {
      take = ties_seen < need;
      ++ties_seen;
    }
    if (take) {
      if (pos < p.budget) out[pos] = (int32_t)(lo + t);
      ++pos;
    }
  }
}

// Fast top-budget selection in three launches (all heads at once):
//   topk_hist_kernel     many workgroups per head: log-linear histogram of the keys (bin = 32 x bit length + the 5
//                        bits after the leading one, 0 for zero; for float keys 32 bins per octave of the value),
//                        monotone in the key. Decode routing fills it in its pool kernel instead.
//   topk_compact_kernel  many workgroups per head: each finds the bin b* holding the budget-th largest key from the
//                        histogram (workgroup 0 records it), then writes indices of keys above b* to `sel` and
//                        (key, index) of keys in b* to the candidate list (at most kTopCand kept; the count goes on),
//                        one atomic per wave and list
//   topk_final_kernel    per head: the need = budget - above best candidates by (key desc, index asc) -- a
//                        histogram of the next 10 key bits narrows them to one sub-bin, whose candidates are ranked
//                        pairwise -- then all chosen keys through an LDS bitmap of the eligible range, emitted
//                        ascending; when the candidates overflowed or the range is too long for the bitmap,
//                        topk_radix_head instead
constexpr int kTopChunk = 4096;       // keys per histogram / compaction workgroup (256 threads x 16)
constexpr int kTopCand = 2048;        // candidates kept per head
constexpr int kTopBitmapBits = 262144;
constexpr int kTopSub = kTopThreads;  // sub-bins of the threshold bin in topk_final_kernel (one per thread)
static_assert(kTopCand <= 32767, "candidate indices fit int16");

// The 10 key bits below the ones top_bin looks at: monotone within one bin (every bin but the two clamped float bins
// holds keys that agree on those higher bits).
BB_DEV int top_sub_key(uint64_t v, bool float_keys) {
  if (!v) return 0;
  if (float_keys) return (int)(((uint32_t)v >> 8) & 1023u);
  const int lz = __clzll((long long)v);
  return (int)(((v << lz) >> 48) & 1023u);
}

struct TopWs {
  uint32_t* hist;     // [heads][kTopBins]
  TopMeta* meta;      // [heads]
  int32_t* sel;       // [heads][n]
  uint64_t* candv;    // [heads][kTopCand]
  int32_t* candi;     // [heads][kTopCand]
};

__global__ __launch_bounds__(256) void topk_hist_kernel(RoutesParams p, TopWs w) {
  __shared__ uint32_t h[kTopBins];
  const int head = blockIdx.y, tid = threadIdx.x;
  int64_t lo, cnt;
  top_range(p, lo, cnt);
  for (int b = tid; b < kTopBins; b += 256) h[b] = 0;
  __syncthreads();
  const uint64_t* P = p.pooled + (int64_t)head * p.pstride + lo;
  const bool fk = p.float_keys != 0;
  const int64_t t0 = (int64_t)blockIdx.x * kTopChunk;
  for (int e = tid; e < kTopChunk; e += 256)
    if (t0 + e < cnt) atomicAdd(&h[top_bin(P[t0 + e], fk)], 1u);
  __syncthreads();
  for (int b = tid; b < kTopBins; b += 256)
    if (h[b]) atomicAdd(&w.hist[(int64_t)head * kTopBins + b], h[b]);
}

// The bin b* that holds the budget-th largest key of one head, from its histogram (all 256 threads of the workgroup
// call it): above = keys in higher bins, need = budget - above. With fewer keys than the budget, b* = 0 and every
// key is taken (need = the zero keys).
struct TopPick {
  int bstar, above, need;
};
BB_DEV TopPick top_pick(const uint32_t* __restrict__ hist, uint32_t budget, uint32_t* part, TopPick* s_pick) {
  constexpr int PER = (kTopBins + 255) / 256;  // bins per thread, taken from the top
  const int tid = threadIdx.x;
  uint32_t c[PER], sum = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int b = kTopBins - 1 - (PER * tid + k);
    c[k] = b >= 0 ? hist[b] : 0u;
    sum += c[k];
  }
  if (tid == 0) *s_pick = TopPick{-1, 0, 0};
  uint32_t total;
  const uint32_t incl = block_incl_scan<256>(sum, part, total);  // over threads, top bins first
  const uint32_t before = incl - sum;
  if (before < budget && incl >= budget) {  // the budget-th largest key lies in this thread's bins
    uint32_t cum = before;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if (cum + c[k] >= budget) {
        *s_pick = TopPick{kTopBins - 1 - (PER * tid + k), (int)cum, (int)(budget - cum)};
        break;
      }
      cum += c[k];
    }
  }
  __syncthreads();
  TopPick r = *s_pick;
  if (r.bstar < 0) {  // fewer keys than the budget: all of them
    const uint32_t zeros = hist[0];
    r = TopPick{0, (int)(total - zeros), (int)zeros};
  }
  return r;
}

__global__ __launch_bounds__(256) void topk_compact_kernel(RoutesParams p, TopWs w) {
  constexpr int PER = kTopChunk / 256;
  __shared__ uint32_t part[256];
  __shared__ uint32_t wcnt[2][4], wbase[2];
  __shared__ TopPick s_pick;
  const int head = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  int64_t lo, cnt;
  top_range(p, lo, cnt);
  const int64_t t0 = (int64_t)blockIdx.x * kTopChunk;
  if (t0 >= cnt) return;  // uniform per workgroup; workgroup 0 always stays when there is any key
  // the chunk's keys are loaded first, so that their latency overlaps the threshold search over the histogram
  const bool fk = p.float_keys != 0;
  const uint64_t* P = p.pooled + (int64_t)head * p.pstride + lo;
  uint64_t v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t t = t0 + 256 * k + tid;
    v[k] = t < cnt ? P[t] : 0;
  }
  const TopPick pk = top_pick(w.hist + (int64_t)head * kTopBins, (uint32_t)p.budget, part, &s_pick);
  TopMeta* m = w.meta + head;
  if (blockIdx.x == 0 && tid == 0) {
    m->bstar = pk.bstar;
    m->above = pk.above;
    m->need = pk.need;
  }
  int bin[PER];
  uint32_t ns = 0, nc = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t t = t0 + 256 * k + tid;
    bin[k] = t < cnt ? top_bin(v[k], fk) : -1;
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    ns += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(bin[k] > pk.bstar));
    nc += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(bin[k] == pk.bstar));
  }
  // one atomic per workgroup and list for the whole chunk (the per-head counters are shared by every chunk)
  const int wave = tid >> 6;
  if (lane == 0) {
    wcnt[0][wave] = ns;
    wcnt[1][wave] = nc;
  }
  __syncthreads();
  if (tid == 0) {
    const uint32_t ts = wcnt[0][0] + wcnt[0][1] + wcnt[0][2] + wcnt[0][3];
    const uint32_t tc = wcnt[1][0] + wcnt[1][1] + wcnt[1][2] + wcnt[1][3];
    wbase[0] = ts ? atomicAdd(&m->nsel, ts) : 0u;
    wbase[1] = tc ? atomicAdd(&m->ncand, tc) : 0u;
  }
  __syncthreads();
  uint32_t base_s = wbase[0], base_c = wbase[1];
  for (int w = 0; w < wave; ++w) {
    base_s += wcnt[0][w];
    base_c += wcnt[1][w];
  }
  int32_t* sel = w.sel + (int64_t)head * p.pstride;
  uint64_t* candv = w.candv + (int64_t)head * kTopCand;
  int32_t* candi = w.candi + (int64_t)head * kTopCand;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint64_t bs = __builtin_amdgcn_ballot_w64(bin[k] > pk.bstar), bc = __builtin_amdgcn_ballot_w64(bin[k] == pk.bstar);
    const uint32_t below_s = __builtin_amdgcn_mbcnt_hi((uint32_t)(bs >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bs, 0u));
    const uint32_t below_c = __builtin_amdgcn_mbcnt_hi((uint32_t)(bc >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bc, 0u));
    const int32_t ix = (int32_t)(lo + t0 + 256 * k + tid);
    if (bin[k] > pk.bstar) sel[base_s + below_s] = ix;
    if (bin[k] == pk.bstar && base_c + below_c < (uint32_t)kTopCand) {
      candv[base_c + below_c] = v[k];
      candi[base_c + below_c] = ix;
    }
    base_s += (uint32_t)__builtin_popcountll(bs);
    base_c += (uint32_t)__builtin_popcountll(bc);
  }
}

__global__ __launch_bounds__(kTopThreads) void topk_final_kernel(RoutesParams p, TopWs w) {
  __shared__ uint64_t cv[kTopCand];
  __shared__ int32_t ci[kTopCand];
  __shared__ uint32_t bits[kTopBitmapBits / 32];
  __shared__ uint32_t scan[kTopThreads / 64];
  __shared__ uint32_t sub[kTopSub];
  __shared__ int16_t tie_list[kTopCand];
  __shared__ int s_sub[3];  // s*, candidates still needed from s*, length of the s* list
  const int head = blockIdx.x, tid = threadIdx.x;
  int64_t lo, cnt;
  top_range(p, lo, cnt);
  const TopMeta m = w.meta[head];
  if (m.ncand > (uint32_t)kTopCand || cnt > kTopBitmapBits) {
    topk_radix_head(p, head);
    return;
  }
  const int nc = (int)m.ncand;
  const int words = (int)((cnt + 31) / 32);
  for (int i = tid; i < nc; i += kTopThreads) {
    cv[i] = w.candv[(int64_t)head * kTopCand + i];
    ci[i] = w.candi[(int64_t)head * kTopCand + i];
  }
  for (int i = tid; i < words; i += kTopThreads) bits[i] = 0u;
  __syncthreads();
  // Chosen candidates: fewer than `need` others beat them (larger value, or equal value and lower index). Inside
  // bin b* the next 10 bits of the key order the candidates further (top_sub_key): a histogram of those finds the
  // sub-bin s* of the need-th largest candidate; candidates above s* are chosen, and only the ones in s* are ranked
  // against each other. The clamped float bins (their keys span several octaves) rank every candidate instead.
  const bool fk = p.float_keys != 0;
  const bool refine = !(fk && (m.bstar == 1 || m.bstar == kTopBins - 1));
  int need2 = m.need, sstar = -1;
  if (refine) {
    for (int i = tid; i < kTopSub; i += kTopThreads) sub[i] = 0u;
    if (tid == 0) {  // need = 0 (every key above b*): no sub-bin, nothing more to choose
      s_sub[0] = kTopSub;
      s_sub[1] = 0;
      s_sub[2] = 0;
    }
    __syncthreads();
    for (int i = tid; i < nc; i += kTopThreads) atomicAdd(&sub[top_sub_key(cv[i], fk)], 1u);
    __syncthreads();
    // thread t owns sub-bin kTopSub - 1 - t (top first): inclusive scan of the counts
    const uint32_t c = sub[kTopSub - 1 - tid];
    uint32_t tot;
    const uint32_t incl = block_incl_scan<kTopThreads>(c, scan, tot);
    if (incl - c < (uint32_t)m.need && incl >= (uint32_t)m.need) {
      s_sub[0] = kTopSub - 1 - tid;
      s_sub[1] = m.need - (int)(incl - c);
    }
    __syncthreads();
    sstar = s_sub[0];
    need2 = s_sub[1];
    // candidates above s* are chosen; the ones in s* go to a short list
    for (int i = tid; i < nc; i += kTopThreads) {
      const int sk = top_sub_key(cv[i], fk);
      if (sk > sstar) atomicOr(&bits[(ci[i] - lo) >> 5], 1u << ((ci[i] - lo) & 31));
      else if (sk == sstar) tie_list[atomicAdd(&s_sub[2], 1)] = i;
    }
    __syncthreads();
  }
  const int nr = refine ? s_sub[2] : nc;
  for (int r = tid; r < nr; r += kTopThreads) {
    const int i = refine ? tie_list[r] : r;
    const uint64_t v = cv[i];
    const int32_t ix = ci[i];
    int rank = 0;
    for (int q = 0; q < nr; ++q) {
      const int j = refine ? tie_list[q] : q;
      rank += (cv[j] > v) || (cv[j] == v && ci[j] < ix);
    }
    if (rank < need2) atomicOr(&bits[(ix - lo) >> 5], 1u << ((ix - lo) & 31));
  }
  for (uint32_t i = tid; i < m.nsel; i += kTopThreads) {
    const int32_t ix = w.sel[(int64_t)head * p.pstride + i];
    atomicOr(&bits[(ix - lo) >> 5], 1u << ((ix - lo) & 31));
  }
  __syncthreads();
  // ascending emission: each thread a contiguous run of words, exclusive scan of their bit counts
  const int per = (words + kTopThreads - 1) / kTopThreads;
  const int w0 = tid * per, w1 = w0 + per < words ? w0 + per : words;
  uint32_t mine = 0;
  for (int x = w0; x < w1; ++x) mine += __builtin_popcount(bits[x]);
  uint32_t chosen;
  uint32_t pos = block_incl_scan<kTopThreads>(mine, scan, chosen) - mine;
  int32_t* out = p.out_idx + (int64_t)head * p.budget;
  for (int x = w0; x < w1; ++x) {
    uint32_t b = bits[x];
    while (b) {
      const int bit = __builtin_ctz(b);
      b &= b - 1;
      if (pos < (uint32_t)p.budget) out[pos] = (int32_t)(lo + 32 * x + bit);
      ++pos;
    }
  }
  // fewer chosen keys than the budget (a short eligible range): the remaining slots read -1
  for (uint32_t i = chosen + tid; i < (uint32_t)p.budget; i += kTopThreads) out[i] = -1;
}

template <int D>
hipError_t launch_routes_d(RoutesParams& p, const RouteGeom& g, float* pmax, uint64_t* psum, float* invz,
                           const TopWs& tw, hipStream_t stream) {
  const int nbkv = p.B * p.Hkv;
  const dim3 sgrid(g.n_kb1, g.row_blocks, nbkv);
  // fp16 scores (8x finer rounding than bf16) are computed in the reference order directly
  if (p.f16)
    hipLaunchKernelGGL((scores_kernel<D, true>), sgrid, dim3(256), 0, stream, p, g, pmax);
  else if (D == 128 && !p.scores_reference_order) {
    const int nw = g.rows <= 64 ? 2 : (g.rows <= 128 ? 4 : 8);  // waves of 32 rows per workgroup
    const dim3 mgrid(g.n_kb1, (g.rows + 32 * nw - 1) / (32 * nw), nbkv);
    if (nw == 2) hipLaunchKernelGGL((scores_mfma_kernel<128, 2>), mgrid, dim3(128), 0, stream, p, g, pmax);
    else if (nw == 4) hipLaunchKernelGGL((scores_mfma_kernel<128, 4>), mgrid, dim3(256), 0, stream, p, g, pmax);
    else hipLaunchKernelGGL((scores_mfma_kernel<128, 8>), mgrid, dim3(512), 0, stream, p, g, pmax);
  } else
    hipLaunchKernelGGL((scores_kernel<D, false>), sgrid, dim3(256), 0, stream, p, g, pmax);
  hipLaunchKernelGGL(rowmax_kernel, dim3(g.rows, nbkv), dim3(64), 0, stream, p, g, pmax);
  if (p.f16) hipLaunchKernelGGL(rowsum_kernel<true>, dim3(g.n_kb2, nbkv, g.sum_splits), dim3(256), 0, stream, p, g, psum);
  else hipLaunchKernelGGL(rowsum_kernel<false>, dim3(g.n_kb2, nbkv, g.sum_splits), dim3(256), 0, stream, p, g, psum);
  hipLaunchKernelGGL(invz_kernel, dim3(g.rows, nbkv), dim3(64), 0, stream, p, g, psum, invz, tw.hist,
                     reinterpret_cast<uint32_t*>(tw.meta));
  const dim3 pgrid((unsigned)((p.n + kPoolKeys - 1) / kPoolKeys), p.B * p.H);
  if (p.f16) hipLaunchKernelGGL(pooled_kernel<true>, pgrid, dim3(256), 0, stream, p, g, invz);
  else hipLaunchKernelGGL(pooled_kernel<false>, pgrid, dim3(256), 0, stream, p, g, invz);
  if (p.budget > 0) {
    int64_t lo = p.sink < p.n ? (p.sink > 0 ? p.sink : 0) : p.n, hi = p.n - p.window < p.n ? p.n - p.window : p.n;
    const int64_t cnt = hi > lo ? hi - lo : 0;
    const unsigned chunks = (unsigned)((cnt + kTopChunk - 1) / kTopChunk);
    const int heads = p.B * p.H;
    hipLaunchKernelGGL(topk_hist_kernel, dim3(chunks, heads), dim3(256), 0, stream, p, tw);
    hipLaunchKernelGGL(topk_compact_kernel, dim3(chunks, heads), dim3(256), 0, stream, p, tw);
    hipLaunchKernelGGL(topk_final_kernel, dim3(heads), dim3(kTopThreads), 0, stream, p, tw);
  }
  return hipGetLastError();
}

RouteGeom geom(int64_t n, int H, int Hkv, int B, int r) {
  RouteGeom g;
  g.G = H / Hkv;
  g.rows = g.G * r;
  g.row_blocks = (g.rows + kMaxRows - 1) / kMaxRows;
  // Longer key chunks per scores workgroup while the grid keeps at least 256 workgroups (one per CU): each workgroup
  // stages its Q rows and bound weights once, so fewer, longer workgroups spend less on that (128K routes, interleaved
  // A/B: 0.885 ms with 16 blocks, 0.812 with 64, 0.793 with 128; the scores are the same)
  const int64_t nbkv = (int64_t)(B > 0 ? B : 1) * Hkv;
  g.iters = kScoreIters;
  while (g.iters < 128) {
    const int64_t chunks = (n + kScoreKeys * 2 * g.iters - 1) / (kScoreKeys * 2 * g.iters);
    if (chunks * g.row_blocks * nbkv < 256) break;
    g.iters *= 2;
  }
  g.n_kb1 = (int)((n + kScoreKeys * g.iters - 1) / (kScoreKeys * g.iters));
  g.n_kb2 = (int)((n + kSumKeys - 1) / kSumKeys);
  g.ns = (n + 7) & ~(int64_t)7;
  // rowsum: about 8 workgroups per CU (2048) per KV-head set, slices of at least 16 rows (4 per wave)
  const int blocks = g.n_kb2 * Hkv > 0 ? g.n_kb2 * Hkv : 1;
  int splits = (2048 + blocks - 1) / blocks;
  const int max_splits = (g.rows + 15) / 16;
  splits = splits < 1 ? 1 : (splits > max_splits ? max_splits : splits);
  g.sum_rows = (((g.rows + splits - 1) / splits) + 3) & ~3;
  g.sum_splits = (g.rows + g.sum_rows - 1) / g.sum_rows;
  return g;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t top_ws_bytes(int64_t n, size_t heads) {
  return align256(heads * kTopBins * 4) + align256(heads * sizeof(TopMeta)) + align256(heads * (size_t)n * 4) +
         align256(heads * kTopCand * 8) + align256(heads * kTopCand * 4);
}

TopWs carve_top_ws(char* w, int64_t n, size_t heads) {
  TopWs t;
  t.hist = reinterpret_cast<uint32_t*>(w); w += align256(heads * kTopBins * 4);
  t.meta = reinterpret_cast<TopMeta*>(w); w += align256(heads * sizeof(TopMeta));
  t.sel = reinterpret_cast<int32_t*>(w); w += align256(heads * (size_t)n * 4);
  t.candv = reinterpret_cast<uint64_t*>(w); w += align256(heads * kTopCand * 8);
  t.candi = reinterpret_cast<int32_t*>(w);
  return t;
}

// Clears the histograms and counters that the top-k kernels accumulate into (pooled_kernel does it for prefill).
__global__ __launch_bounds__(256) void topk_clear_kernel(TopWs w) {
  const int row = blockIdx.x;
  for (int b = threadIdx.x; b < kTopBins; b += 256) w.hist[(int64_t)row * kTopBins + b] = 0u;
  if (threadIdx.x == 0) w.meta[row] = TopMeta{};
}

}  // namespace

size_t topk_workspace_bytes(int64_t stride, int rows) { return top_ws_bytes(stride, (size_t)rows); }

void topk_hist_meta(void* ws, int64_t stride, int rows, uint32_t** hist, uint32_t** meta) {
  const TopWs tw = carve_top_ws(static_cast<char*>(ws), stride, (size_t)rows);
  *hist = tw.hist;
  *meta = reinterpret_cast<uint32_t*>(tw.meta);
}

hipError_t launch_topk_rows(const uint64_t* keys, int rows, int64_t stride, int64_t n, const int64_t* n_dev, int front,
                            int window, int budget, int32_t* out, void* ws, size_t ws_bytes, int flags,
                            hipStream_t stream) {
  if (rows <= 0 || stride <= 0 || budget <= 0 || ws_bytes < topk_workspace_bytes(stride, rows))
    return hipErrorInvalidValue;
  RoutesParams p;
  memset(&p, 0, sizeof(p));
  p.pooled = const_cast<uint64_t*>(keys);
  p.pstride = stride;
  p.n = n < stride ? n : stride;
  p.n_dev = n_dev;
  p.sink = front;
  p.window = window;
  p.budget = budget;
  p.out_idx = out;
  p.float_keys = (flags & kTopFloatKeys) != 0;
  const TopWs tw = carve_top_ws(static_cast<char*>(ws), stride, (size_t)rows);
  // grids cover the largest range the device length can give: [front, stride)
  const int64_t lo = front > 0 ? front : 0;
  const int64_t cnt = stride > lo ? stride - lo : 0;
  const unsigned chunks = (unsigned)((cnt + kTopChunk - 1) / kTopChunk);
  if (!(flags & kTopHistReady)) {
    hipLaunchKernelGGL(topk_clear_kernel, dim3(rows), dim3(256), 0, stream, tw);
    if (chunks > 0) hipLaunchKernelGGL(topk_hist_kernel, dim3(chunks, rows), dim3(256), 0, stream, p, tw);
  }
  if (chunks > 0) hipLaunchKernelGGL(topk_compact_kernel, dim3(chunks, rows), dim3(256), 0, stream, p, tw);
  hipLaunchKernelGGL(topk_final_kernel, dim3(rows), dim3(kTopThreads), 0, stream, p, tw);
  return hipGetLastError();
}

size_t routes_workspace_bytes(int64_t n, int H, int Hkv, int B, int r) {
  RouteGeom g = geom(n, H, Hkv, B, r);
  const size_t nbkv = (size_t)B * Hkv;
  size_t s = 0;
  s += align256(nbkv * g.rows * (size_t)g.ns * 2);        // scores
  s += align256(nbkv * g.n_kb1 * g.rows * 4);             // partial max
  s += align256(nbkv * g.rows * 4);                       // row max
  s += align256(nbkv * g.n_kb2 * g.rows * 8);             // partial sums
  s += align256(nbkv * g.rows * 8);                       // row sums
  s += align256(nbkv * g.rows * 4);                       // 2^40 / Z
  s += align256((size_t)B * H * (size_t)n * 8);           // pooled
  s += top_ws_bytes(n, (size_t)B * H);
  return s;
}

hipError_t launch_routes(RoutesParams& p, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (ws_bytes < routes_workspace_bytes(p.n, p.H, p.Hkv, p.B, p.r)) return hipErrorInvalidValue;
  RouteGeom g = geom(p.n, p.H, p.Hkv, p.B, p.r);
  const size_t nbkv = (size_t)p.B * p.Hkv;
  p.pstride = p.n;
  p.n_dev = nullptr;
  p.float_keys = 0;
  char* w = static_cast<char*>(ws);
  p.scores = reinterpret_cast<uint16_t*>(w); w += align256(nbkv * g.rows * (size_t)g.ns * 2);
  float* pmax = reinterpret_cast<float*>(w); w += align256(nbkv * g.n_kb1 * g.rows * 4);
  p.rowmax = reinterpret_cast<uint32_t*>(w); w += align256(nbkv * g.rows * 4);
  uint64_t* psum = reinterpret_cast<uint64_t*>(w); w += align256(nbkv * g.n_kb2 * g.rows * 8);
  p.rowsum = reinterpret_cast<uint64_t*>(w); w += align256(nbkv * g.rows * 8);
  float* invz = reinterpret_cast<float*>(w); w += align256(nbkv * g.rows * 4);
  p.pooled = reinterpret_cast<uint64_t*>(w); w += align256((size_t)p.B * p.H * (size_t)p.n * 8);
  const TopWs tw = carve_top_ws(w, p.n, (size_t)p.B * p.H);
  switch (p.D) {
    case 32: return launch_routes_d<32>(p, g, pmax, psum, invz, tw, stream);
    case 64: return launch_routes_d<64>(p, g, pmax, psum, invz, tw, stream);
    case 128: return launch_routes_d<128>(p, g, pmax, psum, invz, tw, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bb
