// Decode-time kernels for one new query token (gfx950):
//   * split-K sparse decode (kernels/bigger_bird_decode.py of the reference): each route group attends the virtual
//     key list front | window | routed keys of a bf16 / fp16 KV cache, cut into splits that write partial softmax
//     states, and a merge kernel combines them;
//   * fused decode routing (kernels/bigger_bird_route.py): per-chunk scores of all query heads of a KV head against
//     every cached key with softmax statistics, then the pooled (mean over the group) probability per key with the
//     front and window keys masked out. The top-k selection runs on the routes top-k kernels (bb_routes.hip).
// The cache length may come from device memory (`n_dev`), so a captured HIP graph stays valid as the cache grows in a
// fixed-capacity buffer; every grid is sized from host-side bounds that do not depend on it.
#include "bb_common.h"
#include "bb_internal.h"
#include "bb_topk.h"

namespace bb {
namespace {

template <bool F16>
BB_DEV float elem_to_f32(uint16_t h) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, h);
  else return bf16_to_f32(h);
}
template <bool F16>
BB_DEV uint16_t f32_to_elem(float x) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)x);
  else return f32_to_bf16(x);
}

// fp32 c + a.x b.x + a.y b.y over packed 16-bit pairs (one v_dot2c_f32_{bf16,f16}).
template <bool F16>
BB_DEV float dot2(uint32_t a, uint32_t b, float c) {
  typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_t;
  if constexpr (F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  else return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// The decode kernels read each cached row with the 8 lanes of a key slot. Lane `sub` holds the 16-byte pieces
// sub, sub + 8, ... of the row (element offset piece_off(sub, e0)), so that each load instruction of the slot covers
// whole 128-byte spans of the row: the rows are read once per step, with non-temporal loads (global_load ... nt),
// which stream at about 7.1 TB/s where plain loads reach 6.2-6.3 (16-byte reads over 4 GiB, measured) but which
// fetch whole lines for every instruction, so a lane layout that left half-lines per instruction read them twice.
constexpr int kSlotLanes = 8;
BB_DEV int piece_off(int sub, int e0) { return 8 * (sub + kSlotLanes * e0); }
// Sum over the kSlotLanes = 8 lanes of a key slot (lane bits 0..2), the same value in every lane of the slot, on DPP
// lane moves inside the VALU: quad_perm [1, 0, 3, 2], quad_perm [2, 3, 0, 1], then row_half_mirror (lane i of an
// 8-lane half row reads lane 7 - i, which lies in the other quad and holds that quad's sum). The additions pair the
// same values as a butterfly over lane xor 1, 2, 4, and each lane adds the pair in either order, so every lane holds
// the same bits. (__shfl_xor goes through the LDS crossbar, ds_bpermute, with a wait per round.)
template <int CTRL>
BB_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
BB_DEV float slot_sum8(float v) {
  static_assert(kSlotLanes == 8, "the DPP pattern reduces 8-lane slots");
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  return v;
}
// One round of slot_reduce_scatter over the N heads still held in v[0..N): with N > 1 the lane keeps the upper or
// the lower half (its lane bit for this round) and adds the partner's partials of that half; with N = 1 it adds the
// partner's partial of the one head.
template <int N, int CTRL>
BB_DEV void rs_round(float (&v)[8], bool upper) {
  if constexpr (N == 1) {
    v[0] += dpp_mov<CTRL>(v[0]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float keep = upper ? v[N / 2 + i] : v[i];
      const float send = upper ? v[i] : v[N / 2 + i];
      v[i] = keep + dpp_mov<CTRL>(send);
    }
  }
}
// Reduce-scatter of G per-lane partial sums (G = 1, 2, 4 or 8 heads) over the 8 lanes of a key slot: lane `sub` ends
// with the slot's total for head sub >> (3 - log2 G), each head held by 8 / G lanes with the same bits. The rounds
// pair lane sub with 7 - sub (row_half_mirror), sub ^ 2 and sub ^ 1; the first log2 G of them halve the heads a lane
// holds by lane bit 4, 2 and 1. Every lane's partial of a head enters its total once: the union of sub's quad and
// 7 - sub's quad is the whole slot.
template <int G>
BB_DEV float slot_reduce_scatter(const float (&p)[G], int sub) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "1, 2, 4 or 8 heads per slot");
  constexpr int G1 = G > 1 ? G / 2 : 1, G2 = G1 > 1 ? G1 / 2 : 1;
  float v[8];
#pragma unroll
  for (int i = 0; i < G; ++i) v[i] = p[i];
  rs_round<G, 0x141>(v, (sub & 4) != 0);
  rs_round<G1, 0x4E>(v, (sub & 2) != 0);
  rs_round<G2, 0xB1>(v, (sub & 1) != 0);
  return v[0];
}
constexpr int log2_heads(int g) { return g >= 8 ? 3 : g >= 4 ? 2 : g >= 2 ? 1 : 0; }
BB_DEV u32x4_t ld16_nt(const uint16_t* p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)); }

// q row of one lane's pieces as packed pairs (DPL 16-bit values, DPL / 2 words).
template <int DPL>
BB_DEV void load_q_pairs(const uint16_t* qrow, int sub, uint32_t (&qw)[DPL / 2]) {
#pragma unroll
  for (int e0 = 0; e0 < DPL / 8; ++e0) {
    const u32x4_t w = ld16(qrow + piece_off(sub, e0));
#pragma unroll
    for (int i = 0; i < 4; ++i) qw[4 * e0 + i] = w[i];
  }
}

BB_DEV int64_t current_length(int64_t n, const int64_t* n_dev, int64_t cap) {
  int64_t v = n_dev ? *n_dev : n;
  if (v > cap) v = cap;
  return v < 0 ? 0 : v;
}

// Position of the step's new row (RowAppend): n - 1 when it is appended (1 <= n <= cap), else -1.
BB_DEV int64_t appended_row(const RowAppend& a, int64_t n, const int64_t* n_dev, int64_t cap) {
  const int64_t v = n_dev ? *n_dev : n;
  return a.knew && v >= 1 && v <= cap ? v - 1 : -1;
}

// The 16-byte pieces of lane `sub` (piece_off) of the new K row of KV head kv (already loaded into kw) and of its V row
// to cache row j: each of the 8 lanes of the key slot that read the row writes its own pieces.
template <int DPL>
BB_DEV void store_appended(const RowAppend& a, int kv, int64_t j, int sub, const u32x4_t (&kw)[DPL / 8]) {
#pragma unroll
  for (int e0 = 0; e0 < DPL / 8; ++e0) {
    st16(a.k + (int64_t)kv * a.sk0 + j * a.sk1 + piece_off(sub, e0), kw[e0]);
    st16(a.v + (int64_t)kv * a.sv0 + j * a.sv1 + piece_off(sub, e0),
         ld16(a.vnew + (int64_t)kv * a.svn + piece_off(sub, e0)));
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Sparse split-K decode. Workgroup (split, route row r): 4 waves, 8 lanes per key (D / 8 values each), 32 key slots,
// two keys per slot and step (their K and V rows in flight together). Route row r holds GR query heads (GR = groups
// for pooled routes [Hkv, R], 1 for per-head routes [H, R]) and reads KV head (r GR) / groups. Virtual key
// j < front -> position j; j < front + window -> n - window + (j - front); otherwise the routed index; positions
// outside [0, n) are skipped (kernels/bigger_bird_decode.py:38-47). The key slots of a wave combine through lane
// shuffles, the four waves through LDS. XS (the fused decode step after its routing pass): every key's score is
// already in the routing workspace (p.xs, [H][xs_stride], log2 units, computed from the same q and K rows), so only
// the V rows are read.
constexpr int kSdThreads = 256;
constexpr float kSdRescale = 8.0f;

template <int D, int GR, bool F16, bool XS>
__global__ __launch_bounds__(kSdThreads) void sparse_decode_kernel(SparseDecodeParams p) {
  constexpr int LPK = kSlotLanes, DPL = D / LPK, KPW = 64 / LPK, SLOTS = kSdThreads / LPK, NW = kSdThreads / 64;
  __shared__ float part_m[NW][GR];
  __shared__ float part_l[NW][GR];
  __shared__ float part_o[NW][GR][D];

  const int split = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kslot = lane / LPK, sub = lane % LPK;
  const int slot = wave * KPW + kslot;
  const int64_t n = current_length(p.n, p.n_dev, p.cap);
  const int64_t jnew = appended_row(p.app, p.n, p.n_dev, p.cap);  // read from the new rows, -1: none
  const int kv = (r * GR) / p.G;
  const int64_t total = (int64_t)p.front + p.window + p.route_k;
  const int64_t j_begin = (int64_t)split * p.split_len;
  const int64_t j_end = j_begin + p.split_len < total ? j_begin + p.split_len : total;

  uint32_t qw[GR][DPL / 2];
  if constexpr (!XS) {
#pragma unroll
    for (int h = 0; h < GR; ++h) load_q_pairs<DPL>(p.q + (int64_t)(r * GR + h) * p.sq, sub, qw[h]);
  }
  float m[GR], l[GR], acc[GR][DPL];
#pragma unroll
  for (int h = 0; h < GR; ++h) {
    m[h] = -1.0e20f;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.0f;
  }
  const int32_t* irow = p.idx + (int64_t)r * p.si0;
  const uint16_t* kbase = p.k + (int64_t)kv * p.sk0;
  const uint16_t* vbase = p.v + (int64_t)kv * p.sv0;
  for (int64_t j0 = j_begin + slot; j0 < j_end; j0 += 2 * SLOTS) {
    int64_t pos[2];
    bool ok[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t j = j0 + u * SLOTS;
      int64_t ps;
      if (j < p.front) ps = j;
      else if (j < (int64_t)p.front + p.window) ps = n - p.window + (j - p.front);
      else ps = j < j_end ? irow[(j - p.front - p.window) * p.si1] : -1;
      ok[u] = j < j_end && ps >= 0 && ps < n;  // the 8 lanes of a key slot agree
      pos[u] = ok[u] ? ps : 0;
    }
    u32x4_t kw[2][DPL / 8], vw[2][DPL / 8];
    float xs[2][GR];  // XS: the keys' scores (log2 units) from the routing pass of the same step
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool fresh = ok[u] && pos[u] == jnew;
      const uint16_t* ks = fresh ? p.app.knew + (int64_t)kv * p.app.skn : kbase + pos[u] * p.sk1;
      const uint16_t* vs = fresh ? p.app.vnew + (int64_t)kv * p.app.svn : vbase + pos[u] * p.sv1;
#pragma unroll
      for (int e0 = 0; e0 < DPL / 8; ++e0) {
        if constexpr (!XS) kw[u][e0] = ld16_nt(ks + piece_off(sub, e0));
        vw[u][e0] = ld16_nt(vs + piece_off(sub, e0));
      }
      if constexpr (XS) {
#pragma unroll
        for (int h = 0; h < GR; ++h) xs[u][h] = p.xs[(int64_t)(r * GR + h) * p.xs_stride + pos[u]];
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (!ok[u]) continue;
      float s[GR];
      if constexpr (!XS) {
        if (pos[u] == jnew) store_appended<DPL>(p.app, kv, jnew, sub, kw[u]);
#pragma unroll
        for (int h = 0; h < GR; ++h) {
          float t = 0.0f;
#pragma unroll
          for (int w = 0; w < DPL / 2; ++w) t = dot2<F16>(qw[h][w], kw[u][w >> 2][w & 3], t);
          s[h] = t;
        }
#pragma unroll
        for (int h = 0; h < GR; ++h) s[h] = slot_sum8(s[h]);
      }
#pragma unroll
      for (int h = 0; h < GR; ++h) {
        float x;
        if constexpr (XS) x = xs[u][h];
        else x = s[h] * p.c;
        if (x > m[h] + kSdRescale) {
          const float alpha = fast_exp2(m[h] - x);
          m[h] = x;
          l[h] *= alpha;
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[h][e] *= alpha;
        }
        const float pr = fast_exp2(x - m[h]);
        l[h] += pr;
#pragma unroll
        for (int e = 0; e < DPL; ++e)
          acc[h][e] = fmaf(pr, elem_to_f32<F16>((uint16_t)(vw[u][e >> 3][(e & 7) >> 1] >> (16 * (e & 1)))), acc[h][e]);
      }
    }
  }
  // combine the 8 key slots of the wave (lane bits 3..5), then the waves through LDS
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
    for (int h = 0; h < GR; ++h) {
      const float mo = __shfl_xor(m[h], off), lo = __shfl_xor(l[h], off);
      const float mn = fmaxf(m[h], mo);
      const float a = fast_exp2(m[h] - mn), b = fast_exp2(mo - mn);
      m[h] = mn;
      l[h] = l[h] * a + lo * b;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[h][e] = acc[h][e] * a + __shfl_xor(acc[h][e], off) * b;
    }
  if (kslot == 0) {
#pragma unroll
    for (int h = 0; h < GR; ++h) {
      if (sub == 0) {
        part_m[wave][h] = m[h];
        part_l[wave][h] = l[h];
      }
#pragma unroll
      for (int e = 0; e < DPL; ++e) part_o[wave][h][piece_off(sub, e >> 3) + (e & 7)] = acc[h][e];
    }
  }
  __syncthreads();
  for (int t = tid; t < GR * D; t += kSdThreads) {
    const int h = t / D, d = t % D;
    float M = -1.0e30f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) M = fmaxf(M, part_m[w2][h]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) {
      const float w = fast_exp2(part_m[w2][h] - M);
      L += w * part_l[w2][h];
      O += w * part_o[w2][h][d];
    }
    float* dst = p.part + ((int64_t)(r * GR + h) * p.n_splits + split) * (D + 2);
    dst[d] = O;
    if (d == 0) {
      dst[D] = M;
      dst[D + 1] = L;
    }
  }
}

// Merge of the splits' partial states of one query head (kernels/bigger_bird_decode.py:104-107).
constexpr int kSdMergeThreads = 256;
template <int D, bool F16>
__global__ __launch_bounds__(kSdMergeThreads) void sparse_merge_kernel(SparseDecodeParams p) {
  constexpr int NG = kSdMergeThreads / D;
  __shared__ float red_m[kSdMergeThreads], red_l[NG], red_o[NG][D];
  const int h = blockIdx.x, t = threadIdx.x, d = t % D, grp = t / D;
  const float* base = p.part + (int64_t)h * p.n_splits * (D + 2);
  float M = -1.0e30f;
  for (int s = t; s < p.n_splits; s += kSdMergeThreads) M = fmaxf(M, base[(int64_t)s * (D + 2) + D]);
  red_m[t] = M;
  __syncthreads();
  for (int w = kSdMergeThreads / 2; w > 0; w >>= 1) {
    if (t < w) red_m[t] = fmaxf(red_m[t], red_m[t + w]);
    __syncthreads();
  }
  M = red_m[0];
  float L = 0.0f, O = 0.0f;
  constexpr int U = 8;  // splits per step: their loads are in flight together
  for (int s0 = grp; s0 < p.n_splits; s0 += U * NG) {
    float mv[U], lv[U], ov[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * NG;
      const float* row = base + (int64_t)(s < p.n_splits ? s : 0) * (D + 2);
      mv[u] = s < p.n_splits ? row[D] : -1.0e30f;
      lv[u] = row[D + 1];
      ov[u] = row[d];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float w = s0 + u * NG < p.n_splits ? fast_exp2(mv[u] - M) : 0.0f;
      L += w * lv[u];
      O += w * ov[u];
    }
  }
  red_o[grp][d] = O;
  if (d == 0) red_l[grp] = L;
  __syncthreads();
  if (grp == 0) {
    float lt = 0.0f, ot = 0.0f;
#pragma unroll
    for (int g2 = 0; g2 < NG; ++g2) {
      lt += red_l[g2];
      ot += red_o[g2][d];
    }
    p.out[(int64_t)h * p.so + d] = f32_to_elem<F16>(ot / fmaxf(lt, 1.0e-30f));
  }
  // the step's length advance: no workgroup of this kernel reads the length
  if (p.n_advance && h == 0 && t == 0) {
    const int64_t n = *p.n_advance;
    if (n >= 1 && n <= p.cap) *p.n_advance = n + p.advance;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Decode routing, pass 1 (kernels/bigger_bird_route.py:24-52): workgroup (split, KV head) scores its key range for
// the G query heads (fp32, log2 units, to S [H, cap]) and keeps each head's running (max, sum) per key slot: the
// slot's 8 lanes reduce their partial dot products scatter-wise, so that each lane ends with one head's score and
// keeps that head's state. The slots combine into one (max, sum) per head and split. Each key slot takes eight keys
// per step (all rows in flight: 16 KB per wave; four keys measured 2 us slower per sparse step at 131072 tokens,
// twelve or sixteen spill).
// Split 0 also clears the KV head's top-k histogram and counters, which the pool pass fills.
constexpr int kRsKeysPerSlot = 8;
template <int D, int G, bool F16>
__global__ __launch_bounds__(kSdThreads) void route_scores_kernel(DecodeRouteParams p) {
  constexpr int LPK = kSlotLanes, DPL = D / LPK, KPW = 64 / LPK, SLOTS = kSdThreads / LPK;
  __shared__ float part_m[SLOTS][G];
  __shared__ float part_l[SLOTS][G];
  const int split = blockIdx.x, kv = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kslot = lane / LPK, sub = lane % LPK;
  const int slot = wave * KPW + kslot;
  if (p.top_hist && split == 0) {
    for (int b = tid; b < kTopBins; b += kSdThreads) p.top_hist[(int64_t)kv * kTopBins + b] = 0u;
    if (tid < kTopMetaWords) p.top_meta[(int64_t)kv * kTopMetaWords + tid] = 0u;
  }
  const int64_t n = current_length(p.n, p.n_dev, p.cap);
  const int64_t jnew = appended_row(p.app, p.n, p.n_dev, p.cap);  // read from the new row, -1: none
  const int64_t j_begin = (int64_t)split * p.split_len;
  const int64_t j_end = j_begin + p.split_len < n ? j_begin + p.split_len : n;
  uint32_t qw[G][DPL / 2];
#pragma unroll
  for (int h = 0; h < G; ++h) load_q_pairs<DPL>(p.q + (int64_t)(kv * G + h) * p.sq, sub, qw[h]);
  // after the slot reduction lane sub holds head myh's score; the first of the head's 8 / G lanes writes it
  constexpr int HSH = 3 - log2_heads(G);
  const int myh = sub >> HSH;
  const bool writer = (sub & ((1 << HSH) - 1)) == 0;
  float m = -1.0e20f, l = 0.0f;  // head myh's running (max, sum) over this slot's keys
  constexpr int U = kRsKeysPerSlot;
  const uint16_t* kbase = p.k + (int64_t)kv * p.sk0;
  float* srow = p.scores + (int64_t)(kv * G + myh) * p.cap;
  for (int64_t j0 = j_begin + slot; j0 < j_end; j0 += U * SLOTS) {
    u32x4_t kw[U][DPL / 8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + u * SLOTS < j_end ? j0 + u * SLOTS : j0;
      const uint16_t* ks = j == jnew ? p.app.knew + (int64_t)kv * p.app.skn : kbase + j * p.sk1;
#pragma unroll
      for (int e0 = 0; e0 < DPL / 8; ++e0) kw[u][e0] = ld16_nt(ks + piece_off(sub, e0));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + u * SLOTS;
      if (j >= j_end) break;  // the 8 lanes of a key slot agree
      if (j == jnew) store_appended<DPL>(p.app, kv, jnew, sub, kw[u]);
      float sc[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < DPL / 2; ++w) t = dot2<F16>(qw[h][w], kw[u][w >> 2][w & 3], t);
        sc[h] = t;
      }
      const float x = slot_reduce_scatter<G>(sc, sub) * p.c;
      if (writer) srow[j] = x;
      // l 2^(m - mn) + 2^(x - mn) with mn = max(m, x), on one exponential: one of the two factors is 2^0 = 1
      const float dx = x - m;
      const float e = fast_exp2(-fabsf(dx));
      l = dx <= 0.0f ? l + e : fmaf(l, e, 1.0f);
      m = fmaxf(m, x);
    }
  }
  if (writer) {
    part_m[slot][myh] = m;
    part_l[slot][myh] = l;
  }
  __syncthreads();
  if (tid < G) {
    const int h = tid;
    float M = -1.0e20f;
    for (int s2 = 0; s2 < SLOTS; ++s2) M = fmaxf(M, part_m[s2][h]);
    float L = 0.0f;
    for (int s2 = 0; s2 < SLOTS; ++s2) L += part_l[s2][h] * fast_exp2(part_m[s2][h] - M);
    const int64_t o = ((int64_t)kv * p.n_splits + split) * G + h;
    p.stat_m[o] = M;
    p.stat_l[o] = L;
  }
}

BB_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
BB_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
  return v;
}

// Decode routing, pass 2 (kernels/bigger_bird_route.py:55-80): merges each head's split statistics (one wave per
// head, lanes over the splits), then per key p = mean over the group of 2^(s - M) / Z; keys outside
// [front, n - window) get -1. With top-k keys it also writes the order-preserving 64-bit keys (fp32 bits of p) and
// adds the eligible keys to the KV head's top-k histogram (LDS counts, then one atomic per non-empty bin).
// 8 keys per thread (2048 per workgroup): 1.1 us less per sparse decode step at 131072 tokens than 4 (fewer
// workgroups repeat the split-statistics merge and flush a histogram); 2 and 16 measured slower
constexpr int kRpThreads = 256, kRpPer = 8, kRpKeys = kRpThreads * kRpPer;
template <int G>
__global__ __launch_bounds__(kRpThreads) void route_pool_kernel(DecodeRouteParams p) {
  __shared__ float sm[G], sinv[G];
  __shared__ uint32_t hist[kTopBins];
  const int kv = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t n = current_length(p.n, p.n_dev, p.cap);
  const bool top = p.keys && p.top_hist;
  if (top)
    for (int b = tid; b < kTopBins; b += kRpThreads) hist[b] = 0u;
  for (int h = wave; h < G; h += kRpThreads / 64) {
    const float* pm = p.stat_m + (int64_t)kv * p.n_splits * G + h;
    const float* pl = p.stat_l + (int64_t)kv * p.n_splits * G + h;
    float M = -1.0e20f;
    for (int s = lane; s < p.n_splits; s += 64) M = fmaxf(M, pm[(int64_t)s * G]);
    M = wave_max(M);
    float L = 0.0f;
    for (int s = lane; s < p.n_splits; s += 64) L += pl[(int64_t)s * G] * fast_exp2(pm[(int64_t)s * G] - M);
    L = wave_sum(L);
    if (lane == 0) {
      sm[h] = M;
      sinv[h] = 1.0f / fmaxf(L, 1.0e-30f);
    }
  }
  __syncthreads();
  const int64_t hi = n - p.window;
#pragma unroll
  for (int u = 0; u < kRpPer; ++u) {
    const int64_t j = (int64_t)blockIdx.x * kRpKeys + u * kRpThreads + tid;
    if (j < p.cap) {
      const bool eligible = j >= p.front && j < hi;
      float pr = -1.0f;
      if (eligible) {
        float sc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) sc[h] = p.scores[(int64_t)(kv * G + h) * p.cap + j];
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < G; ++h) acc += fast_exp2(sc[h] - sm[h]) * sinv[h];
        pr = acc / (float)G;
      }
      p.probs[(int64_t)kv * p.cap + j] = pr;
      if (p.keys) {
        const uint64_t key = float_key(pr);
        p.keys[(int64_t)kv * p.cap + j] = key;
        if (top && eligible) atomicAdd(&hist[top_bin(key, true)], 1u);
      }
    }
  }
  if (top) {
    __syncthreads();
    for (int b = tid; b < kTopBins; b += kRpThreads)
      if (hist[b]) atomicAdd(&p.top_hist[(int64_t)kv * kTopBins + b], hist[b]);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Cache compaction for kv_evict (modal_rd/attention.py:250-257): dst[h, i, :] = src[h, idx[h, i], :] for rows of
// D 16-bit elements (16 bytes per thread), and the float priorities -> order-preserving 64-bit keys for the top-k.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src, int64_t ss0, int64_t ss1,
                                                          int64_t n_src, const int64_t* __restrict__ idx, int64_t si0,
                                                          int m, int D, uint16_t* __restrict__ dst, int64_t sd0,
                                                          int64_t sd1) {
  const int h = blockIdx.y, cpr = D / 8;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)m * cpr) return;
  const int i = (int)(e / cpr), c = (int)(e % cpr);
  const int64_t row = idx[(int64_t)h * si0 + i];
  const bool ok = row >= 0 && row < n_src;  // an index outside the source gives a zero row
  st16(dst + (int64_t)h * sd0 + (int64_t)i * sd1 + 8 * c,
       ok ? ld16(src + (int64_t)h * ss0 + row * ss1 + 8 * c) : u32x4_t{0, 0, 0, 0});
}

// One decode step's cache append: row n = *n_dev of every KV head of k and of v (strides head, token) takes the new
// rows knew / vnew [heads, D] (head strides), then *n_dev advances by n_inc. One workgroup, so every thread reads the
// length before thread 0 moves it. A length at or past the capacity writes nothing and leaves the length as it is.
__global__ __launch_bounds__(256) void kv_append_kernel(uint16_t* __restrict__ k, int64_t sk0, int64_t sk1,
                                                        uint16_t* __restrict__ v, int64_t sv0, int64_t sv1,
                                                        const uint16_t* __restrict__ knew, int64_t skn,
                                                        const uint16_t* __restrict__ vnew, int64_t svn, int heads, int D,
                                                        int64_t cap, int64_t* __restrict__ n_dev, int64_t n_inc) {
  const int64_t n = *n_dev;
  const int cpr = D / 8;
  if (n >= 0 && n < cap) {
    for (int e = threadIdx.x; e < 2 * heads * cpr; e += 256) {
      const int which = e / (heads * cpr), r = e % (heads * cpr), h = r / cpr, c = r % cpr;
      const uint16_t* src = which ? vnew + (int64_t)h * svn : knew + (int64_t)h * skn;
      uint16_t* dst = which ? v + (int64_t)h * sv0 + n * sv1 : k + (int64_t)h * sk0 + n * sk1;
      st16(dst + 8 * c, ld16(src + 8 * c));
    }
  }
  __syncthreads();  // every thread has read n
  if (threadIdx.x == 0 && n >= 0 && n < cap) *n_dev = n + n_inc;
}

__global__ __launch_bounds__(256) void f32_keys_kernel(const float* __restrict__ vals, int64_t sv0, int64_t n,
                                                       uint64_t* __restrict__ keys) {
  const int r = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  const float x = vals[(int64_t)r * sv0 + j];
  keys[(int64_t)r * n + j] = float_key(x);  // NaN and x <= 0 sort last
}

// ---------------------------------------------------------------------------------------------------------------
// Greedy token choice of a decode step (modal_rd/graph_decode.py:201-202): the index of the largest logit of one row,
// torch.argmax semantics (a NaN is larger than every number, the first index wins ties). One 1024-thread workgroup,
// so a captured decode step holds no multi-workgroup reduction (and no counters to clear between replays).
constexpr int kAmThreads = 1024;

BB_DEV bool am_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

template <typename T, int EPU>  // element type (float, bf16 / fp16 bits), elements per load
__global__ __launch_bounds__(kAmThreads) void argmax_kernel(const T* __restrict__ x, int64_t n, int kind,
                                                            int64_t* __restrict__ out) {
  __shared__ float wv[kAmThreads / 64];
  __shared__ int wi[kAmThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto value = [&](T raw) -> float {
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(float, raw);
    else return kind == 2 ? (float)__builtin_bit_cast(_Float16, (uint16_t)raw) : bf16_to_f32((uint16_t)raw);
  };
  float bv = -__builtin_huge_valf();
  int bi = 0x7fffffff;
  const int64_t units = n / EPU;
  for (int64_t u = tid; u < units; u += kAmThreads) {
    T e[EPU];
    if constexpr (EPU > 1) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(x + u * EPU);
      __builtin_memcpy(e, &w, sizeof(w));
    } else {
      e[0] = x[u];
    }
#pragma unroll
    for (int k = 0; k < EPU; ++k) {
      const float v = value(e[k]);
      const int i = (int)(u * EPU + k);
      if (am_better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
  }
  for (int64_t i = units * EPU + tid; i < n; i += kAmThreads) {
    const float v = value(x[i]);
    if (am_better(v, (int)i, bv, bi)) {
      bv = v;
      bi = (int)i;
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (am_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    wv[wave] = bv;
    wi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kAmThreads / 64; ++w)
      if (am_better(wv[w], wi[w], bv, bi)) {
        bv = wv[w];
        bi = wi[w];
      }
    out[0] = bi == 0x7fffffff ? 0 : bi;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// RMSNorm of a decode step's hidden rows with the arithmetic of HF LlamaRMSNorm on a 16-bit model: x in fp32,
// r = rsqrt(mean(x^2) + eps), y = round(x r) to the model dtype, out = round(w y). One 256-thread workgroup per
// row, 8 values per 16-byte load (D % 8 == 0, D <= 8192). RES: x is first replaced by round(x + res) (the residual
// add of a decoder layer, as a 16-bit tensor add computes it), which is also written to sum.
constexpr int kRnThreads = 256;
constexpr int kRnMaxD = 8192;
// One row's arithmetic, shared by rms_norm_kernel and gemv_kernel's norm prologue: a 256-thread workgroup, thread t
// holding the 16-byte units t, t + 256, ... of the row. sumr (may be null) receives round(x + res); emit(c, v) takes
// the 8 normalised values at element c.
template <bool F16, bool RES, typename Emit>
BB_DEV void norm_row(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ rr, const uint16_t* __restrict__ w,
                     int D, float eps, float* red, uint16_t* __restrict__ sumr, Emit emit) {
  const int tid = threadIdx.x;
  constexpr int kMaxUnits = kRnMaxD / 8 / kRnThreads;  // 16-byte units per thread at D = 8192
  u32x4_t xv[kMaxUnits];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kMaxUnits; ++u) {
    const int c = (u * kRnThreads + tid) * 8;
    xv[u] = c < D ? ld16(xr + c) : u32x4_t{0, 0, 0, 0};
    if (RES && c < D) {
      const u32x4_t rv = ld16(rr + c);
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        uint32_t pair = 0;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const float a = elem_to_f32<F16>((uint16_t)(xv[u][e2] >> (16 * hb)));
          const float b = elem_to_f32<F16>((uint16_t)(rv[e2] >> (16 * hb)));
          pair |= (uint32_t)f32_to_elem<F16>(a + b) << (16 * hb);
        }
        xv[u][e2] = pair;
      }
      if (sumr) st16(sumr + c, xv[u]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = elem_to_f32<F16>((uint16_t)(xv[u][e >> 1] >> (16 * (e & 1))));
      ss = fmaf(f, f, ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  const float r = rsqrtf(total * (1.0f / (float)D) + eps);
#pragma unroll
  for (int u = 0; u < kMaxUnits; ++u) {
    const int c = (u * kRnThreads + tid) * 8;
    if (c >= D) break;
    const u32x4_t wv = ld16(w + c);
    u32x4_t o;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t pair = 0;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        const int e = 2 * e2 + hb;
        const float f = elem_to_f32<F16>((uint16_t)(xv[u][e >> 1] >> (16 * (e & 1))));
        const float y = elem_to_f32<F16>(f32_to_elem<F16>(f * r));
        const float wf = elem_to_f32<F16>((uint16_t)(wv[e >> 1] >> (16 * (e & 1))));
        pair |= (uint32_t)f32_to_elem<F16>(wf * y) << (16 * hb);
      }
      o[e2] = pair;
    }
    emit(c, o);
  }
}

template <bool F16, bool RES>
__global__ __launch_bounds__(kRnThreads) void rms_norm_kernel(const uint16_t* __restrict__ x, int64_t sx,
                                                              const uint16_t* __restrict__ res, int64_t sr,
                                                              const uint16_t* __restrict__ w, int D, float eps,
                                                              uint16_t* __restrict__ out, int64_t so,
                                                              uint16_t* __restrict__ sum, int64_t ssum) {
  __shared__ float red[kRnThreads / 64];
  const int64_t row = blockIdx.x;
  uint16_t* orow = out + row * so;
  norm_row<F16, RES>(x + row * sx, RES ? res + row * sr : nullptr, w, D, eps, red, RES ? sum + row * ssum : nullptr,
                     [&](int c, u32x4_t v) { st16(orow + c, v); });
}

// out = round(round(silu(g)) u) elementwise over n values (n % 8 == 0, 16-byte aligned): the arithmetic of
// F.silu(g) * u on 16-bit tensors (silu in fp32 as g / (1 + exp(-g)), rounded; the product in fp32, rounded), i.e.
// the activation of a Llama MLP between its gate / up and down projections.
template <bool F16>
BB_DEV u32x4_t silu_mul8(u32x4_t gv, u32x4_t uv) {
  u32x4_t o;
#pragma unroll
  for (int e2 = 0; e2 < 4; ++e2) {
    uint32_t pair = 0;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const float x = elem_to_f32<F16>((uint16_t)(gv[e2] >> (16 * hb)));
      const float a = elem_to_f32<F16>(f32_to_elem<F16>(x / (1.0f + expf(-x))));
      const float b = elem_to_f32<F16>((uint16_t)(uv[e2] >> (16 * hb)));
      pair |= (uint32_t)f32_to_elem<F16>(a * b) << (16 * hb);
    }
    o[e2] = pair;
  }
  return o;
}

template <bool F16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                       int64_t n, uint16_t* __restrict__ out) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= n) return;
  st16(out + c, silu_mul8<F16>(ld16(g + c), ld16(u + c)));
}

// ---------------------------------------------------------------------------------------------------------------
// One token through a linear layer, y[N] = W[N, K] x[K] (16-bit W rows of stride sw; fp32 accumulation, y rounded
// to the model dtype): the decode step's projections, HBM-bound on streaming W once. A workgroup is 4 waves; each
// group of KS waves takes R rows, the KS waves of a group taking consecutive parts of K; lane l of a wave takes the
// 16-byte chunks l, l + 64, ... of its part of the rows (512 values per step; 1 KB of a row per load instruction,
// non-temporal since W is read once per token: 5.6 against 5.2 TB/s over 8 layers' weights), with A steps of its R
// rows' loads in flight, and x is staged once per workgroup in LDS (after the first steps' W loads are issued, so the staging hides
// under their latency). Each lane sums its share of a row with v_dot2c_f32_{bf16,f16}, the wave sums the lanes, and
// the KS waves' sums are added in LDS in wave order. NORM: x is the RMSNorm of a hidden row (RES: of hid + res, the
// sum also written to `sum` by workgroup 0), computed by every workgroup with rms_norm_kernel's arithmetic (so the
// product is bit-identical to bb_add_rms_norm / bb_rms_norm followed by the plain GEMV). GLU: W holds 2N rows, gate rows [0, N) above up rows [N, 2N) (a Llama MLP's fused
// gate / up projection); a wave takes R / 2 outputs i with both their rows i and N + i, and writes
// round(round(silu(g)) u) of the rounded g and u (silu_mul_kernel's arithmetic): the MLP's activation input.
constexpr int kGvWaves = 4;
constexpr int kGvMaxK = 16384;  // x staged in 32 KB of LDS
template <bool F16, bool GLU, bool NORM, bool RES, int R, int A, int KS>
__global__ __launch_bounds__(64 * kGvWaves) void gemv_kernel(const uint16_t* __restrict__ w, int64_t sw, int N, int K,
                                                              const uint16_t* __restrict__ x, GemvNorm nm,
                                                              uint16_t* __restrict__ y, int rounds) {
  static_assert(!GLU || R % 2 == 0, "GLU rows come in (gate, up) pairs");
  static_assert(kGvWaves % KS == 0, "K parts split the workgroup's waves evenly");
  static_assert(!NORM || 64 * kGvWaves == kRnThreads, "the norm prologue runs on rms_norm_kernel's thread layout");
  constexpr int OUTS = GLU ? R / 2 : R;   // outputs per group of KS waves and round
  constexpr int GROUPS = kGvWaves / KS;   // wave groups per workgroup
  __shared__ float red[kGvWaves];
  __shared__ __attribute__((aligned(16))) uint16_t xs[kGvMaxK];
  __shared__ float part[2][KS > 1 ? kGvWaves : 1][R];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / KS, kp = wave % KS;
  const int gid = blockIdx.x * GROUPS + grp, ngroups = gridDim.x * GROUPS;  // wave group, all wave groups
  const int kc = K / 8;                                     // 16-byte chunks per row
  const int steps = ((kc + 63) / 64 + KS - 1) / KS;         // 512-value steps per K part (every wave the same)
  const int sbeg = kp * steps;
  const int total = rounds * steps;                         // this wave's (round, step) sequence
  // row r of round k: output group gid + k ngroups (rows past the end read the last row; their outputs are not
  // stored)
  auto row = [&](int k, int r) -> const uint16_t* {
    const int o = (gid + k * ngroups) * OUTS + (GLU ? r / 2 : r);
    const int oc = o < N ? o : N - 1;
    return w + (int64_t)(GLU ? oc + (r & 1) * N : oc) * sw;
  };
  int lk = 0, lst = 0;  // next (round, step) to load
  auto load = [&](u32x4_t (&dst)[R]) {
    const int c = (sbeg + lst) * 64 + lane;
#pragma unroll
    for (int r = 0; r < R; ++r) dst[r] = c < kc ? ld16_nt(row(lk, r) + 8 * c) : u32x4_t{0, 0, 0, 0};
    if (++lst == steps) {
      lst = 0;
      ++lk;
    }
  };
  u32x4_t buf[A][R];
#pragma unroll
  for (int a = 0; a < A; ++a)
    if (a < total) load(buf[a]);
  const int xchunks = KS * steps * 64;  // chunks of x the waves read (zero past K)
  if constexpr (NORM) {
    norm_row<F16, RES>(x, nm.res, nm.w, K, nm.eps, red, RES && blockIdx.x == 0 ? nm.sum : nullptr,
                       [&](int c, u32x4_t v) { *reinterpret_cast<u32x4_t*>(&xs[c]) = v; });
    for (int c = kc + tid; c < xchunks; c += 64 * kGvWaves)
      *reinterpret_cast<u32x4_t*>(&xs[8 * c]) = u32x4_t{0, 0, 0, 0};
  } else {
    for (int c = tid; c < xchunks; c += 64 * kGvWaves)
      *reinterpret_cast<u32x4_t*>(&xs[8 * c]) = c < kc ? ld16(x + 8 * c) : u32x4_t{0, 0, 0, 0};
  }
  __syncthreads();
  float acc[R] = {};
  int ck = 0, cst = 0;  // (round, step) being summed
  for (int t0 = 0; t0 < total; t0 += A) {
#pragma unroll
    for (int a = 0; a < A; ++a) {
      if (t0 + a < total) {
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(&xs[8 * ((sbeg + cst) * 64 + lane)]);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r] = dot2<F16>(buf[a][r][e], xv[e], acc[r]);
        if (t0 + a + A < total) load(buf[a]);
        if (++cst == steps) {  // round ck done: sum the lanes, then the K parts, and store its outputs
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
          if constexpr (KS > 1) {
            if (lane == 0) {
#pragma unroll
              for (int r = 0; r < R; ++r) part[ck & 1][wave][r] = acc[r];
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float s2 = part[ck & 1][grp * KS][r];
#pragma unroll
              for (int j = 1; j < KS; ++j) s2 += part[ck & 1][grp * KS + j][r];
              acc[r] = s2;
            }
          }
          const int out0 = (gid + ck * ngroups) * OUTS;
          if (kp == 0 && lane < OUTS && out0 + lane < N) {
            float v = acc[0];  // acc[lane] with a static index
#pragma unroll
            for (int r = 1; r < OUTS; ++r) v = lane == r ? acc[GLU ? 2 * r : r] : v;
            if constexpr (GLU) {
              float u = acc[1];
#pragma unroll
              for (int r = 1; r < OUTS; ++r) u = lane == r ? acc[2 * r + 1] : u;
              const uint32_t gp = f32_to_elem<F16>(v), up = f32_to_elem<F16>(u);
              y[out0 + lane] = (uint16_t)silu_mul8<F16>(u32x4_t{gp, 0, 0, 0}, u32x4_t{up, 0, 0, 0})[0];
            } else {
              y[out0 + lane] = f32_to_elem<F16>(v);
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] = 0.0f;
          cst = 0;
          ++ck;
        }
      }
    }
  }
}

template <int D, int GR, bool F16>
hipError_t launch_sparse_decode_t(const SparseDecodeParams& p, hipStream_t stream) {
  if (p.xs)
    hipLaunchKernelGGL((sparse_decode_kernel<D, GR, F16, true>), dim3(p.n_splits, p.rows), dim3(kSdThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((sparse_decode_kernel<D, GR, F16, false>), dim3(p.n_splits, p.rows), dim3(kSdThreads), 0, stream,
                       p);
  hipLaunchKernelGGL((sparse_merge_kernel<D, F16>), dim3(p.H), dim3(kSdMergeThreads), 0, stream, p);
  return hipGetLastError();
}

template <int D, bool F16>
hipError_t launch_sparse_decode_d(const SparseDecodeParams& p, hipStream_t stream) {
  switch (p.rows == p.H ? 1 : p.G) {
    case 1: return launch_sparse_decode_t<D, 1, F16>(p, stream);
    case 2: return launch_sparse_decode_t<D, 2, F16>(p, stream);
    case 4: return launch_sparse_decode_t<D, 4, F16>(p, stream);
    case 8: return launch_sparse_decode_t<D, 8, F16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D, int G, bool F16>
hipError_t launch_route_t(const DecodeRouteParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((route_scores_kernel<D, G, F16>), dim3(p.n_splits, p.Hkv), dim3(kSdThreads), 0, stream, p);
  hipLaunchKernelGGL(route_pool_kernel<G>, dim3((unsigned)((p.cap + kRpKeys - 1) / kRpKeys), p.Hkv), dim3(kRpThreads),
                     0, stream, p);
  return hipGetLastError();
}

template <int D, bool F16>
hipError_t launch_route_d(const DecodeRouteParams& p, hipStream_t stream) {
  switch (p.H / p.Hkv) {
    case 1: return launch_route_t<D, 1, F16>(p, stream);
    case 2: return launch_route_t<D, 2, F16>(p, stream);
    case 4: return launch_route_t<D, 4, F16>(p, stream);
    case 8: return launch_route_t<D, 8, F16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_sparse_decode(const SparseDecodeParams& p, hipStream_t stream) {
  if (p.n_splits <= 0 || p.rows <= 0) return hipErrorInvalidValue;
  if (p.D == 64) return p.f16 ? launch_sparse_decode_d<64, true>(p, stream) : launch_sparse_decode_d<64, false>(p, stream);
  if (p.D == 128)
    return p.f16 ? launch_sparse_decode_d<128, true>(p, stream) : launch_sparse_decode_d<128, false>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_gather_rows(const uint16_t* src, int64_t ss0, int64_t ss1, int64_t n_src, int heads,
                              const int64_t* idx, int64_t si0, int m, int D, uint16_t* dst, int64_t sd0, int64_t sd1,
                              hipStream_t stream) {
  const int64_t work = (int64_t)m * (D / 8);
  if (work <= 0 || heads <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((work + 255) / 256), heads), dim3(256), 0, stream, src, ss0,
                     ss1, n_src, idx, si0, m, D, dst, sd0, sd1);
  return hipGetLastError();
}

hipError_t launch_kv_append(uint16_t* k, int64_t sk0, int64_t sk1, uint16_t* v, int64_t sv0, int64_t sv1,
                            const uint16_t* knew, int64_t skn, const uint16_t* vnew, int64_t svn, int heads, int D,
                            int64_t cap, int64_t* n_dev, int64_t n_inc, hipStream_t stream) {
  hipLaunchKernelGGL(kv_append_kernel, dim3(1), dim3(256), 0, stream, k, sk0, sk1, v, sv0, sv1, knew, skn, vnew, svn,
                     heads, D, cap, n_dev, n_inc);
  return hipGetLastError();
}

hipError_t launch_argmax(const void* x, int64_t n, int kind, bool vec16, int64_t* out, hipStream_t stream) {
  if (n <= 0 || n > 0x7ffffffe) return hipErrorInvalidValue;
  if (kind == 0) {
    if (vec16)
      hipLaunchKernelGGL((argmax_kernel<uint32_t, 4>), dim3(1), dim3(kAmThreads), 0, stream,
                         static_cast<const uint32_t*>(x), n, kind, out);
    else
      hipLaunchKernelGGL((argmax_kernel<uint32_t, 1>), dim3(1), dim3(kAmThreads), 0, stream,
                         static_cast<const uint32_t*>(x), n, kind, out);
  } else if (vec16) {
    hipLaunchKernelGGL((argmax_kernel<uint16_t, 8>), dim3(1), dim3(kAmThreads), 0, stream,
                       static_cast<const uint16_t*>(x), n, kind, out);
  } else {
    hipLaunchKernelGGL((argmax_kernel<uint16_t, 1>), dim3(1), dim3(kAmThreads), 0, stream,
                       static_cast<const uint16_t*>(x), n, kind, out);
  }
  return hipGetLastError();
}

hipError_t launch_rms_norm(const uint16_t* x, int64_t sx, const uint16_t* res, int64_t sr, int rows, int D,
                           const uint16_t* w, float eps, int f16, uint16_t* out, int64_t so, uint16_t* sum,
                           int64_t ssum, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  if (D <= 0 || D % 8 || D > 8192 || (res != nullptr) != (sum != nullptr)) return hipErrorInvalidValue;
  const dim3 grid(rows), block(kRnThreads);
  if (res) {
    if (f16)
      hipLaunchKernelGGL((rms_norm_kernel<true, true>), grid, block, 0, stream, x, sx, res, sr, w, D, eps, out, so,
                         sum, ssum);
    else
      hipLaunchKernelGGL((rms_norm_kernel<false, true>), grid, block, 0, stream, x, sx, res, sr, w, D, eps, out, so,
                         sum, ssum);
  } else if (f16) {
    hipLaunchKernelGGL((rms_norm_kernel<true, false>), grid, block, 0, stream, x, sx, res, sr, w, D, eps, out, so,
                       sum, ssum);
  } else {
    hipLaunchKernelGGL((rms_norm_kernel<false, false>), grid, block, 0, stream, x, sx, res, sr, w, D, eps, out, so,
                       sum, ssum);
  }
  return hipGetLastError();
}

// Rows per group R = 2, A = 8 steps in flight, K in KS = 2 parts: the fastest of the (R, A, KS) shapes measured for
// Llama-3-8B's decode projections (q/k/v 6144 x 4096, o 4096 x 4096, gate / up 28672 x 4096, down 4096 x 14336:
// 12.2, 10.7, 40.3 and 23.3 us, against 12.0-14.1, 10.8-11.7, 42.3-50.4 and 24.0-31.0 us for (4, 4, 1), (2, 8, 1),
// (4, 2, 4), (4, 4, 4), (2, 4, 4) and (4, 4, 2)).
constexpr int kGvR = 2, kGvA = 8, kGvKS = 2;
constexpr int kGvMaxGroups = 1024;

template <bool F16, bool GLU, bool NORM, bool RES>
hipError_t launch_gemv_t(const uint16_t* w, int64_t sw, int N, int K, const uint16_t* x, const GemvNorm& nm,
                         uint16_t* y, hipStream_t stream) {
  // workgroups: at most kGvMaxGroups; each wave group takes `rounds` output groups, spread so that the last round
  // is as full as the others
  constexpr int outs = kGvWaves / kGvKS * (GLU ? kGvR / 2 : kGvR);  // outputs per workgroup and round
  const int64_t wg_needed = (N + outs - 1) / outs;
  int cap = kGvMaxGroups;
  if (const char* e = getenv("BB_GEMV_CAP")) cap = atoi(e);
  const int rounds = (int)((wg_needed + cap - 1) / cap);
  const unsigned grid = (unsigned)((wg_needed + rounds - 1) / rounds);
  hipLaunchKernelGGL((gemv_kernel<F16, GLU, NORM, RES, kGvR, kGvA, kGvKS>), dim3(grid), dim3(64 * kGvWaves), 0,
                     stream, w, sw, N, K, x, nm, y, rounds);
  return hipGetLastError();
}

template <bool F16, bool GLU>
hipError_t launch_gemv_g(const uint16_t* w, int64_t sw, int N, int K, const uint16_t* x, const GemvNorm* nm,
                         uint16_t* y, hipStream_t stream) {
  if (!nm) return launch_gemv_t<F16, GLU, false, false>(w, sw, N, K, x, GemvNorm{}, y, stream);
  if (nm->res) return launch_gemv_t<F16, GLU, true, true>(w, sw, N, K, x, *nm, y, stream);
  return launch_gemv_t<F16, GLU, true, false>(w, sw, N, K, x, *nm, y, stream);
}

hipError_t launch_gemv(const uint16_t* w, int64_t sw, int N, int K, const uint16_t* x, const GemvNorm* nm, bool glu,
                       int f16, uint16_t* y, hipStream_t stream) {
  if (N <= 0) return hipSuccess;
  if (K <= 0 || K % 8 || K > kGvMaxK || (nm && K > kRnMaxD)) return hipErrorInvalidValue;
  if (f16) return glu ? launch_gemv_g<true, true>(w, sw, N, K, x, nm, y, stream)
                      : launch_gemv_g<true, false>(w, sw, N, K, x, nm, y, stream);
  return glu ? launch_gemv_g<false, true>(w, sw, N, K, x, nm, y, stream)
             : launch_gemv_g<false, false>(w, sw, N, K, x, nm, y, stream);
}

hipError_t launch_silu_mul(const uint16_t* g, const uint16_t* u, int64_t n, int f16, uint16_t* out,
                           hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (n % 8) return hipErrorInvalidValue;
  const unsigned blocks = (unsigned)((n / 8 + 255) / 256);
  if (f16) hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(blocks), dim3(256), 0, stream, g, u, n, out);
  else hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(blocks), dim3(256), 0, stream, g, u, n, out);
  return hipGetLastError();
}

hipError_t launch_f32_keys(const float* vals, int64_t sv0, int rows, int64_t n, uint64_t* keys, hipStream_t stream) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  hipLaunchKernelGGL(f32_keys_kernel, dim3((unsigned)((n + 255) / 256), rows), dim3(256), 0, stream, vals, sv0, n, keys);
  return hipGetLastError();
}

hipError_t launch_decode_route_probs(const DecodeRouteParams& p, hipStream_t stream) {
  if (p.n_splits <= 0 || p.Hkv <= 0 || p.cap <= 0) return hipErrorInvalidValue;
  if (p.D == 64) return p.f16 ? launch_route_d<64, true>(p, stream) : launch_route_d<64, false>(p, stream);
  if (p.D == 128) return p.f16 ? launch_route_d<128, true>(p, stream) : launch_route_d<128, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace bb
