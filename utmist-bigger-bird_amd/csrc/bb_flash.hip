// Sink + causal window + routed sparse flash attention for gfx950 (bf16 MFMA, fp32 online softmax).
//
// Semantics follow kernels/bigger_bird_flash.py:42-96 of the reference: for query row q (absolute position) the
// attended keys are   front:  j < FRONT and j <= q
//                     window: j >= FRONT and q - WINDOW < j <= q
//                     routed: j in idx[bh, group(q)], FRONT <= j <= q - WINDOW
// with one joint softmax over their union; query head bh reads KV head (bh // H) * (H // G) + (bh % H) // G.
//
// Work decomposition (MI355X-first, not the reference's one-program-per-(64 rows, head) grid):
//   * a workgroup of NW waves owns one KV head, HPW of its query heads and R query rows per head (256 query rows in
//     total); every K/V tile staged in LDS is shared by all HPW heads (GQA reuse inside the workgroup);
//   * a wave owns QB blocks of 32 query rows of one head and computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so
//     each lane holds one query's scores: row max and row sum stay in-lane apart from one permlane32 swap with the
//     partner lane holding the other half of the keys;
//   * P never leaves registers: the S^T accumulator layout is the B operand of O^T += V^T P^T once the V^T fragment
//     reads use the matching key permutation, so V is consumed transposed; a one-pass kernel writes V^T [D][N] once
//     per layer, after which K and V^T window tiles stream global->LDS with 16-byte direct loads
//     (global_load_lds_dwordx4, no staging registers) into XOR-swizzled, bank-conflict-free layouts;
//   * window tiles are 64-key aligned and double buffered; only edge tiles evaluate masks;
//   * routed keys differ across the heads of a group, so they are gathered per head into per-head LDS tiles
//     (K rows by direct loads, V rows transposed through registers);
//   * the exponent offset is refreshed only when a tile max exceeds it by more than 2^8, which keeps O rescales off
//     the steady-state path without changing the normalised result;
//   * SPLIT mode (exact tail: window = N, no routes) cuts the key range into chunks and writes (O, m, l) partials that
//     launch_flash_merge combines, so 256 tail rows still fill all 256 CUs;
//   * blockIdx -> (KV head, row tile) is XCD-aware: consecutive workgroups on one XCD walk neighbouring row tiles of
//     one KV head, so their windows overlap in that XCD's L2.
#include "bb_common.h"
#include "bb_flash_tiles.h"
#include "bb_internal.h"

namespace bb {
namespace {

// One 64-key tile for one wave: S^T = K Q^T, online softmax, O^T += V^T P^T.
template <bool F16, int D, int QB, bool MASKED, typename Mask>
BB_DEV void tile_step(WaveState<D, QB>& st, const uint16_t* kl, const uint16_t* vt, int lane, float c, int64_t qabs0,
                      int64_t step, const Mask& mask) {
  const int h = lane >> 5, li = lane & 31;
  f32x16_t s[QB][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[qb][kb] = f32x16_t{};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int dk = 0; dk < D / 16; ++dk) {
      const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(kl + k_off<D>(32 * kb + li, 2 * dk + h)));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[qb][kb] = mma32<F16>(a, st.qf[qb][dk], s[qb][kb]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  bf16x8_t pk[QB][2][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if constexpr (MASKED) {
      const auto mrow = mask.row(qabs0 + (32 * qb + li) * step);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
          if (!mrow(kk)) s[qb][kb][r] = -__builtin_huge_valf();
        }
    }
    float mx = fmaxf(s[qb][0][0], s[qb][1][0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[qb][0][r], s[qb][1][r]));
    mx = xhalf_max(mx);
    const float mt = mx * c;
    const bool need = mt > st.m[qb] + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float alpha = need ? fast_exp2(st.m[qb] - mt) : 1.0f;
      if (need) st.m[qb] = mt;
      st.l[qb] *= alpha;
#pragma unroll
      for (int dv = 0; dv < D / 32; ++dv)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.o[qb][dv][r] *= alpha;
    }
    const float nm = -st.m[qb];
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = fast_exp2(fmaf(s[qb][kb][8 * u + e], c, nm));
          sum += p[e];
        }
        pk[qb][kb][u] = as_bf16x8(u32x4_t{pack2<F16>(p[0], p[1]), pack2<F16>(p[2], p[3]), pack2<F16>(p[4], p[5]),
                                          pack2<F16>(p[6], p[7])});
      }
    }
    st.l[qb] += sum;
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int unit = 2 * (2 * kb + u) + h;
#pragma unroll
      for (int dv = 0; dv < D / 32; ++dv) {
        const int d = 32 * dv + li;
        const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(vt + vt_off(d, unit)));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) st.o[qb][dv] = mma32<F16>(a, pk[qb][kb][u], st.o[qb][dv]);
      }
    }
  }
}

template <bool F16, int D, int NW, int HPW, bool SPLIT, bool HAS_MASK>
__global__ __launch_bounds__(64 * NW, 1) void flash_kernel(FlashParams p) {
  constexpr int QB = 256 / 32 / NW;  // 32-row query blocks per wave (256 query rows per workgroup)
  constexpr int WPH = NW / HPW;      // waves per head
  constexpr int RW = 32 * QB;        // rows per wave
  constexpr int R = WPH * RW;        // rows per head per workgroup
  constexpr int kThreads = 64 * NW;
  static_assert(QB >= 1 && WPH >= 1, "workgroup shape");
  constexpr int kWinElems = 2 * Layout<D>::kTileElems;
  constexpr int kRouteElems = HPW * Layout<D>::kTileElems;
  constexpr int kLdsElems = kWinElems > kRouteElems ? kWinElems : kRouteElems;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsElems];
  __shared__ int32_t route_keys[HPW][kTileKeys];
  __shared__ int wg_batches[NW];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, li = lane & 31;

  // ---- work item ----
  const int lanes_total = p.n_kvbh * p.head_splits;
  const int per_lane = p.row_tiles * p.n_chunks;
  int lane_id, within;
  const int bid = blockIdx.x;
  if (p.remap) {
    const int x = bid & 7, s = bid >> 3;
    lane_id = x + 8 * (s / per_lane);
    within = s % per_lane;
  } else {
    lane_id = bid % lanes_total;
    within = bid / lanes_total;
  }
  const int rt = p.row_tiles - 1 - within / p.n_chunks;
  const int chunk = within % p.n_chunks;
  const int kvbh = lane_id / p.head_splits, hsplit = lane_id % p.head_splits;
  const int batch = kvbh / p.Hkv_pb;
  const int bh_base = batch * p.H + (kvbh % p.Hkv_pb) * p.G + hsplit * HPW;

  const int64_t T_eff = p.row_end < p.T ? p.row_end : p.T;
  const int64_t r0 = (int64_t)rt * R;
  const int64_t r1 = (r0 + R < T_eff ? r0 + R : T_eff) - 1;
  const int64_t qlo = p.offset + r0 * p.pos_step, qhi = p.offset + r1 * p.pos_step;

  const int slot = wave / WPH, rb = wave % WPH;
  const int bh = bh_base + slot;
  const int64_t rw = r0 + (int64_t)RW * rb;
  const bool wave_active = rw <= r1;
  const int64_t qw0 = p.offset + rw * p.pos_step;
  const int64_t qw1 = p.offset + (rw + RW - 1 < r1 ? rw + RW - 1 : r1) * p.pos_step;
  const uint8_t* km = HAS_MASK ? p.key_mask + (int64_t)batch * p.smb : nullptr;

  WaveState<D, QB> st;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t row = rw + 32 * qb + li;
    const uint16_t* qrow = p.q + (int64_t)bh * p.sq0 + row * p.sq1 + 8 * h;
#pragma unroll
    for (int dk = 0; dk < D / 16; ++dk)
      st.qf[qb][dk] = as_bf16x8(row < T_eff ? ld16(qrow + 16 * dk) : u32x4_t{0, 0, 0, 0});
#pragma unroll
    for (int dv = 0; dv < D / 32; ++dv) st.o[qb][dv] = f32x16_t{};
    st.m[qb] = -1.0e20f;
    st.l[qb] = 0.0f;
  }

  const uint16_t* kbase = p.k + (int64_t)kvbh * p.sk0;
  const uint16_t* vbase = p.v + (int64_t)kvbh * p.sv0;
  const uint16_t* vtbase = p.vt + (int64_t)kvbh * D * p.np;

  // ---- tile ranges (64-aligned): front tiles then window tiles ----
  const int64_t front_end = p.front < qhi + 1 ? p.front : qhi + 1;
  int64_t wlo = qlo - p.window + 1;
  if (wlo < 0) wlo = 0;
  int64_t kmin = 0, kmax = qhi;
  if (SPLIT) {
    kmin = (int64_t)chunk * p.key_chunk;
    const int64_t ke = kmin + p.key_chunk - 1;
    if (ke < kmax) kmax = ke;
  }
  int64_t f0 = 0, f1 = front_end > 0 ? (front_end + kTileKeys - 1) / kTileKeys : 0;
  int64_t w0 = wlo / kTileKeys, w1 = qhi / kTileKeys + 1;
  if (w0 <= f1) {
    f1 = 0;
    w0 = 0;
  }
  const int64_t c0 = kmin / kTileKeys, c1 = kmax / kTileKeys + 1;
  if (f0 < c0) f0 = c0;
  if (f1 > c1) f1 = c1;
  if (f1 < f0) f1 = f0;
  if (w0 < c0) w0 = c0;
  if (w1 > c1) w1 = c1;
  if (w1 < w0) w1 = w0;
  const int64_t n1 = f1 - f0, ntiles = n1 + (w1 - w0);

  auto tile_k = [&](int i) { return smem + i * Layout<D>::kTileElems; };
  auto tile_v = [&](int i) { return smem + i * Layout<D>::kTileElems + Layout<D>::kKElems; };
  auto tile_pos = [&](int64_t t) { return (t < n1 ? f0 + t : w0 + (t - n1)) * kTileKeys; };

  if (ntiles > 0) {
    issue_window_tile<D, NW>(tile_k(0), tile_v(0), kbase, p.sk1, vtbase, p.np, tile_pos(0), p.N, wave, lane);
    wait_vm();
    __syncthreads();
    for (int64_t t = 0; t < ntiles; ++t) {
      const int cur = (int)(t & 1);
      const int64_t k0 = tile_pos(t);
      if (t + 1 < ntiles)
        issue_window_tile<D, NW>(tile_k(cur ^ 1), tile_v(cur ^ 1), kbase, p.sk1, vtbase, p.np, tile_pos(t + 1), p.N,
                                 wave, lane);
      if (wave_active) {
        const int64_t k1 = k0 + kTileKeys - 1;
        const bool skip = k0 > qw1 || (k0 >= p.front && k1 <= qw0 - p.window);
        if (!skip) {
          const bool full = !HAS_MASK && k1 <= qw0 && k1 < p.N && (k1 < p.front || k0 >= qw1 - p.window + 1);
          const WindowMask wm{k0, p.N, p.front, p.window, km};
          if (full)
            tile_step<F16, D, QB, false>(st, tile_k(cur), tile_v(cur), lane, p.c, qw0, p.pos_step, wm);
          else
            tile_step<F16, D, QB, true>(st, tile_k(cur), tile_v(cur), lane, p.c, qw0, p.pos_step, wm);
        }
      }
      wait_vm();
      __syncthreads();
    }
  }

  // ---- routed keys (never in SPLIT mode): per-head gathered tiles, all waves in lockstep ----
  if (!SPLIT && p.route_k > 0) {
    int64_t g_first = qlo / p.route_chunk, g_last = qhi / p.route_chunk;
    if (g_last >= p.n_groups) g_last = p.n_groups - 1;
    uint16_t* kl = tile_k(slot);
    uint16_t* vt = tile_v(slot);
    const int wih = rb;  // wave index within its head
    for (int64_t g = g_first; g <= g_last; ++g) {
      const bool in_group = wave_active && qw0 / p.route_chunk <= g && qw1 / p.route_chunk >= g;
      const int32_t* irow = p.idx + (int64_t)bh * p.si0 + g * p.si1;
      int my_batches = 0;
      if (in_group) {
        for (int s0 = 0; s0 < p.route_k; s0 += kTileKeys) {
          const int sl = s0 + lane;
          const int64_t key = sl < p.route_k ? irow[sl * p.si2] : -1;
          const bool ok = key >= p.front && key < p.N && key <= qw1 - p.window;
          if (__builtin_amdgcn_ballot_w64(ok)) my_batches = s0 / kTileKeys + 1;
        }
      }
      if (lane == 0) wg_batches[wave] = my_batches;
      __syncthreads();
      int nb = 0, head_nb = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        nb = nb > wg_batches[w] ? nb : wg_batches[w];
        if (w / WPH == slot) head_nb = head_nb > wg_batches[w] ? head_nb : wg_batches[w];
      }
      // the head's highest valid row decides which keys are gathered
      const int64_t head_q1 = qhi;
      for (int bi = 0; bi < nb; ++bi) {
        const bool head_work = bi < head_nb;
        if (head_work && wih == 0) {
          const int sl = bi * kTileKeys + lane;
          const int64_t key = sl < p.route_k ? irow[sl * p.si2] : -1;
          const bool ok = key >= p.front && key < p.N && key <= head_q1 - p.window;
          route_keys[slot][lane] = ok ? (int32_t)key : -1;
        }
        __syncthreads();
        if (head_work) {
          // K rows: direct loads; this head's WPH waves split the blocks
          for (int b = wih; b < Layout<D>::kBlocks; b += WPH) {
            const int e = b * 512 + 8 * lane;
            const int row = e / D, sl2 = (e % D) / 8;
            const int chk = sl2 ^ (row & (Layout<D>::CPR - 1));
            const int32_t key = route_keys[slot][row];
            lds_dma16(kbase + (int64_t)(key >= 0 ? key : 0) * p.sk1 + 8 * chk, kl + b * 512);
          }
          // V rows -> V^T through registers: units of 4 keys x 8 d
          constexpr int CPR = D / 8;
          for (int u = lane + 64 * wih; u < (kTileKeys / 4) * CPR; u += 64 * WPH) {
            const int bq = u % CPR, a = u / CPR;
            u32x4_t vr[4];
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
              const int32_t key = route_keys[slot][4 * a + s2];
              vr[s2] = key >= 0 ? ld16(vbase + (int64_t)key * p.sv1 + 8 * bq) : u32x4_t{0, 0, 0, 0};
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int w = e >> 1;
              const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
              const uint32_t lo = __builtin_amdgcn_perm(vr[1][w], vr[0][w], sel);
              const uint32_t hi = __builtin_amdgcn_perm(vr[3][w], vr[2][w], sel);
              const int d = 8 * bq + e;
              *reinterpret_cast<u32x2_t*>(vt + vt_off(d, 2 * (a >> 2) + (a & 1)) + 4 * ((a >> 1) & 1)) = u32x2_t{lo, hi};
            }
          }
        }
        wait_vm();
        __syncthreads();
        if (head_work && bi < my_batches) {
          const RoutedMask rm{route_keys[slot], p.window, p.route_chunk, g, km};
          tile_step<F16, D, QB, true>(st, kl, vt, lane, p.c, qw0, p.pos_step, rm);
        }
        __syncthreads();
      }
      __syncthreads();
    }
  }

  // ---- epilogue ----
  if (!wave_active) return;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t row = rw + 32 * qb + li;
    const float lt = xhalf_sum(st.l[qb]);
    if (row >= T_eff) continue;
    if constexpr (SPLIT) {
      const int64_t base = ((int64_t)chunk * p.BH + bh) * p.T + row;
      float* po = p.part_o + base * D;
#pragma unroll
      for (int dv = 0; dv < D / 32; ++dv)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d0 = 32 * dv + 8 * g4 + 4 * h;
          *reinterpret_cast<f32x4_t*>(po + d0) =
              f32x4_t{st.o[qb][dv][4 * g4], st.o[qb][dv][4 * g4 + 1], st.o[qb][dv][4 * g4 + 2], st.o[qb][dv][4 * g4 + 3]};
        }
      if (h == 0) {
        p.part_ml[2 * base] = st.m[qb];
        p.part_ml[2 * base + 1] = lt;
      }
    } else {
      float inv = 1.0f / fmaxf(lt, 1.0e-20f);
      if (HAS_MASK && !km[row + p.offset]) inv = 0.0f;
      uint16_t* orow = p.out + (int64_t)bh * p.so0 + row * p.so1;
#pragma unroll
      for (int dv = 0; dv < D / 32; ++dv)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d0 = 32 * dv + 8 * g4 + 4 * h;
          const u32x2_t w = {pack2<F16>(st.o[qb][dv][4 * g4] * inv, st.o[qb][dv][4 * g4 + 1] * inv),
                             pack2<F16>(st.o[qb][dv][4 * g4 + 2] * inv, st.o[qb][dv][4 * g4 + 3] * inv)};
          *reinterpret_cast<u32x2_t*>(orow + d0) = w;
        }
    }
  }
}

// Combine split partials: one wave per (head, row); lanes cover D.
template <bool F16, int D>
__global__ __launch_bounds__(256) void flash_merge_kernel(FlashParams p) {
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t rows = p.row_end < p.T ? p.row_end : p.T;
  if (item >= (int64_t)p.BH * rows) return;
  const int bh = (int)(item / rows);
  const int64_t row = item % rows;
  float M = -1.0e30f;
  for (int c = 0; c < p.n_chunks; ++c) {
    const int64_t base = ((int64_t)c * p.BH + bh) * p.T + row;
    M = fmaxf(M, p.part_ml[2 * base]);
  }
  float L = 0.0f;
  constexpr int PER = (D + 63) / 64;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.0f;
  for (int c = 0; c < p.n_chunks; ++c) {
    const int64_t base = ((int64_t)c * p.BH + bh) * p.T + row;
    const float w = fast_exp2(p.part_ml[2 * base] - M);
    L += w * p.part_ml[2 * base + 1];
    const float* po = p.part_o + base * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int d = lane + 64 * i;
      if (d < D) acc[i] += w * po[d];
    }
  }
  float inv = 1.0f / fmaxf(L, 1.0e-20f);
  if (p.key_mask && !p.key_mask[(int64_t)(bh / p.H) * p.smb + row + p.offset]) inv = 0.0f;
  uint16_t* orow = p.out + (int64_t)bh * p.so0 + row * p.so1;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    if (d < D) orow[d] = to16<F16>(acc[i] * inv);
  }
}

// V [n_kvbh][N][D] (strided) -> V^T [n_kvbh][D][np], zero columns for keys >= N; keys of every 16-key group in
// vt_key_pos order.
template <int D>
__global__ __launch_bounds__(256) void transpose_v_kernel(const uint16_t* __restrict__ v, int64_t sv0, int64_t sv1,
                                                          int64_t N, int64_t np, uint16_t* __restrict__ vt) {
  __shared__ uint16_t tile[kTileKeys][D + 2];
  const int64_t k0 = (int64_t)blockIdx.x * kTileKeys;
  const int kvbh = blockIdx.y;
  const uint16_t* src = v + (int64_t)kvbh * sv0;
  for (int e = threadIdx.x; e < kTileKeys * (D / 8); e += 256) {
    const int row = e / (D / 8), c8 = e % (D / 8);
    const int64_t pos = k0 + row;
    const u32x4_t w = pos < N ? ld16(src + pos * sv1 + 8 * c8) : u32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tile[row][8 * c8 + 2 * i] = (uint16_t)(w[i] & 0xffffu);
      tile[row][8 * c8 + 2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
  }
  __syncthreads();
  uint16_t* dst = vt + (int64_t)kvbh * D * np;
  for (int e = threadIdx.x; e < D * (kTileKeys / 8); e += 256) {
    const int d = e / (kTileKeys / 8), c8 = e % (kTileKeys / 8);
    // row position 8 c8 + j holds key vt_key_pos(8 c8 + j) (the permutation is its own inverse)
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ka = vt_key_pos(8 * c8 + 2 * i);  // positions 2i and 2i + 1 hold consecutive keys
      w[i] = (uint32_t)tile[ka][d] | ((uint32_t)tile[ka + 1][d] << 16);
    }
    st16(dst + (int64_t)d * np + k0 + 8 * c8, u32x4_t{w[0], w[1], w[2], w[3]});
  }
}

template <int D, int NW, int HPW, bool SPLIT>
hipError_t launch_dhs(const FlashParams& p, hipStream_t stream) {
  const int64_t items = (int64_t)p.n_kvbh * p.head_splits * p.row_tiles * p.n_chunks;
  if (items <= 0) return hipSuccess;
  if (items > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)items), block(64 * NW);
  if (p.f16) {
    if (p.key_mask) hipLaunchKernelGGL((flash_kernel<true, D, NW, HPW, SPLIT, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_kernel<true, D, NW, HPW, SPLIT, false>), grid, block, 0, stream, p);
  } else {
    if (p.key_mask) hipLaunchKernelGGL((flash_kernel<false, D, NW, HPW, SPLIT, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_kernel<false, D, NW, HPW, SPLIT, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

template <int D, int NW>
hipError_t launch_dw(const FlashParams& p, int hpw, bool split, hipStream_t stream) {
  switch (hpw) {
    case 4: return split ? launch_dhs<D, NW, 4, true>(p, stream) : launch_dhs<D, NW, 4, false>(p, stream);
    case 2: return split ? launch_dhs<D, NW, 2, true>(p, stream) : launch_dhs<D, NW, 2, false>(p, stream);
    case 1: return split ? launch_dhs<D, NW, 1, true>(p, stream) : launch_dhs<D, NW, 1, false>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int D>
hipError_t launch_d(const FlashParams& p, int hpw, bool split, hipStream_t stream) {
  return launch_dw<D, 8>(p, hpw, split, stream);
}

}  // namespace

hipError_t launch_flash(const FlashParams& p, int D, int hpw, bool split, hipStream_t stream) {
  switch (D) {
    case 32: return launch_d<32>(p, hpw, split, stream);
    case 64: return launch_d<64>(p, hpw, split, stream);
    case 128: return launch_d<128>(p, hpw, split, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_flash_merge(const FlashParams& p, int D, hipStream_t stream) {
  const int64_t rows = p.row_end < p.T ? p.row_end : p.T;
  const int64_t items = (int64_t)p.BH * rows;
  if (items <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((items + 3) / 4);
  switch (D) {
    case 32: if (p.f16) hipLaunchKernelGGL((flash_merge_kernel<true, 32>), dim3(blocks), dim3(256), 0, stream, p); else hipLaunchKernelGGL((flash_merge_kernel<false, 32>), dim3(blocks), dim3(256), 0, stream, p); break;
    case 64: if (p.f16) hipLaunchKernelGGL((flash_merge_kernel<true, 64>), dim3(blocks), dim3(256), 0, stream, p); else hipLaunchKernelGGL((flash_merge_kernel<false, 64>), dim3(blocks), dim3(256), 0, stream, p); break;
    case 128: if (p.f16) hipLaunchKernelGGL((flash_merge_kernel<true, 128>), dim3(blocks), dim3(256), 0, stream, p); else hipLaunchKernelGGL((flash_merge_kernel<false, 128>), dim3(blocks), dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_transpose_v(const uint16_t* v, int64_t sv0, int64_t sv1, int n_kvbh, int64_t N, int64_t np, int D,
                              uint16_t* vt, hipStream_t stream) {
  if (n_kvbh <= 0 || N <= 0) return hipSuccess;
  const dim3 grid((unsigned)(np / kTileKeys), (unsigned)n_kvbh);
  switch (D) {
    case 32: hipLaunchKernelGGL(transpose_v_kernel<32>, grid, dim3(256), 0, stream, v, sv0, sv1, N, np, vt); break;
    case 64: hipLaunchKernelGGL(transpose_v_kernel<64>, grid, dim3(256), 0, stream, v, sv0, sv1, N, np, vt); break;
    case 128: hipLaunchKernelGGL(transpose_v_kernel<128>, grid, dim3(256), 0, stream, v, sv0, sv1, N, np, vt); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bb
