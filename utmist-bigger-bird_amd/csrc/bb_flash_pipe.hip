// Ping-pong sink + causal window + routed sparse flash attention for gfx950 (head_dim 128, no token mask): the main
// pass of Bigger Bird v3 prefill at production shape.
//
// Same semantics as bb_flash.hip (kernels/bigger_bird_flash.py:42-96 of the reference). Work decomposition:
//   * a workgroup = 8 waves = the 4 query heads of one KV head x 2 blocks of 32 query rows (64 rows); every K / V^T
//     tile staged in LDS is read by all 8 waves (GQA reuse inside the workgroup). With 2 query heads per KV head a
//     workgroup is 2 heads x 4 row blocks (128 rows), with 1 (MHA) one head x 8 row blocks (256 rows), so the tiles
//     are still shared by all 8 waves;
//   * waves w and w + 4 share a SIMD. Per 64-key tile a wave runs an MFMA phase  (O^T += V^T(t-1) P(t-1)^T,
//     S(t) = K(t) Q^T: 32 MFMAs) and a VALU phase (online softmax of S(t) into P(t)), separated by workgroup
//     barriers. Waves 4..7 start one barrier late, so on every SIMD one wave is in its MFMA phase while the other is
//     in its VALU phase: the matrix cores and the VALUs work at the same time instead of in turn;
//   * K and V^T tiles stream global->LDS with 16-byte buffer loads straight into LDS (no staging registers) through a
//     four-stage ring, issued two tiles ahead at the end of a VALU phase; rows past N read as zeros through the buffer
//     resource bounds;
//   * the exponent offset moves only when a probability would exceed 2^8 (O rescales stay rare); tiles without masked
//     elements skip the per-tile maximum unless the row sum says the offset must move;
//   * routed keys differ per head: after the window loop the two waves of a head stream its routed K / V^T tiles into
//     that head's LDS tile, pre-gathered per 64-slot batch by route_tiles_kernel (one route group), or gather the
//     batch's K rows and V rows themselves (several route groups: the GATHER instantiation).
#include "bb_common.h"
#include "bb_flash_tiles.h"
#include "bb_internal.h"

namespace bb {
namespace {

constexpr int PD = 128;                 // head_dim
constexpr int PNW = 8;                  // waves per workgroup
constexpr int PHEADS = 4;               // most query heads per workgroup (HPW = 4, 2 or 1 share each tile)
constexpr int PTE = kTileKeys * PD;     // elements of one K (or V^T) tile
constexpr int PST = 4;                  // ring stages, each a K tile and a V^T tile
constexpr int PBLK = PTE * 2 / 1024;    // 1 KB direct-load blocks per tile (16)
constexpr int PLDS = PST * 2 * PTE;     // 128 KB; the routed phase reuses it as 4 heads x (K + V^T)
constexpr int kRouteCache = 512;        // route slots per head staged in LDS at a time
static_assert(PHEADS * 2 * PTE <= PLDS, "routed tiles fit the ring");

typedef __attribute__((__vector_size__(4 * sizeof(int32_t)))) int32_t i32x4_t;

// Element masks. In the S^T layout lane (li, h) holds, for key half kb of a tile, the keys
// kk = 32 kb + 4 h + j(r), j(r) = 8 (r / 4) + r % 4, r = 0..15; j(r) grows with r, so each of the conditions
// kk <= q - k0 (causal), kk < front - k0 and kk > q - window - k0 selects a prefix or a suffix of r. Masks are
// returned as 16 bits per key half.
BB_DEV uint32_t prefix_upto(int a) {  // bits r with j(r) <= a
  if (a < 0) return 0u;
  if (a >= 27) return 0xFFFFu;
  const int n = 4 * (a >> 3) + ((a & 7) < 3 ? (a & 7) + 1 : 4);
  return (1u << n) - 1u;
}

BB_DEV int clamp_rel(int64_t x) { return (int)(x > 64 ? 64 : (x < -1 ? -1 : x)); }

struct PipeWindowMask {  // front | causal window (nothing when !any)
  int64_t k0, front, window;
  bool any;
  BB_DEV uint32_t bits(int64_t q, int kb, int h) const {
    if (!any) return 0u;
    const int64_t base = k0 + 32 * kb + 4 * h;
    const uint32_t causal = prefix_upto(clamp_rel(q - base));
    const uint32_t fr = prefix_upto(clamp_rel(front - base - 1));
    const uint32_t win = ~prefix_upto(clamp_rel(q - window - base)) & 0xFFFFu;
    return causal & (fr | win);
  }
};

struct PipeRoutedMask {  // gathered key list (-1 = empty): key <= q - window, and q in the list's route group
  const int32_t* keys;
  int64_t window, route_chunk, group;
  BB_DEV uint32_t bits(int64_t q, int kb, int h) const {
    const int64_t lim64 = q / route_chunk == group ? q - window : -1;
    const int lim = lim64 > 0x7fffffff ? 0x7fffffff : (lim64 < -1 ? -1 : (int)lim64);
    uint32_t b = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const i32x4_t k4 = *reinterpret_cast<const i32x4_t*>(keys + 32 * kb + 8 * g + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) b |= (uint32_t)(k4[e] >= 0 && k4[e] <= lim) << (4 * g + e);
    }
    return b;
  }
};

// Direct global->LDS tile loads through buffer resources (one per KV head: rows past N read as zeros, and every
// per-lane offset is a loop-invariant 32-bit value). Block b (1 KB) of a tile is loaded by wave b % 8; its lanes
// land at byte 16 * lane of the block.
struct TileLoader {
  __amdgpu_buffer_rsrc_t krs, vrs;
  uint32_t kvoff, vvoff;    // per-lane byte offsets of this wave's first block
  uint32_t kstep, vstep;    // byte distance between this wave's two blocks (8 blocks apart)
  uint32_t krow_bytes;
  int wave;

  BB_DEV void init(const uint16_t* kbase, int64_t sk1, int64_t N, const uint16_t* vtbase, int64_t np, int w,
                   int lane) {
    wave = w;
    krow_bytes = (uint32_t)(sk1 * 2);
    // num_records is an unsigned 32-bit byte count (passed through int): sizes up to 4 GiB
    krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase), 0, (int)(uint32_t)(N * sk1 * 2), 0x00020000);
    vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vtbase), 0, (int)(uint32_t)(PD * np * 2), 0x00020000);
    // K block b = w + 8i: rows 4b + lane/16, 16-byte chunk (lane%16) ^ (row%16); row%16 does not depend on i
    const int krow = 4 * w + lane / 16;
    kvoff = (uint32_t)krow * krow_bytes + 16u * (uint32_t)((lane % 16) ^ (krow & 15));
    kstep = 32u * krow_bytes;
    // V^T block b = w + 8i: d = 8b + lane/8, 16-byte unit (lane%8) ^ vt_swz(d); vt_swz(d) does not depend on i
    const int d = 8 * w + lane / 8;
    vvoff = (uint32_t)d * (uint32_t)(np * 2) + 16u * (uint32_t)((lane % 8) ^ vt_swz(d));
    vstep = 64u * (uint32_t)(np * 2);
  }
  BB_DEV void tile(uint16_t* kl, uint16_t* vt, int64_t k0) const {
    // The K tile offset goes into the per-lane offset: the buffer range check covers it (and not the scalar
    // offset), so rows past N read as zeros instead of touching memory past the tensor.
    const uint32_t kb = kvoff + (uint32_t)k0 * krow_bytes, vb = (uint32_t)k0 * 2u;
#pragma unroll
    for (int i = 0; i < PBLK / PNW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          krs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                   reinterpret_cast<uintptr_t>(kl + (wave + PNW * i) * 512)),
          16, kb + i * kstep, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < PBLK / PNW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          vrs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                   reinterpret_cast<uintptr_t>(vt + (wave + PNW * i) * 512)),
          16, vvoff, vb + i * vstep, 0, 0);
  }
};

BB_DEV void vm_wait_tile(bool one_tile_in_flight) {
  // vmcnt(4) keeps the most recent tile's 4 loads (2 K + 2 V^T blocks) in flight; vmcnt(0) drains everything
  if (one_tile_in_flight) __builtin_amdgcn_s_waitcnt(0x0F74);
  else __builtin_amdgcn_s_waitcnt(0x0F70);
}

// Workgroup barrier without a memory fence: the tile ring publishes its direct loads with explicit vmcnt waits,
// so the barrier must not drain the loads still in flight for the tile after next (a __syncthreads fence would).
// The wavefront-scope fences emit nothing but keep the compiler from moving memory accesses across it; the
// scheduling barriers keep register arithmetic on its side too (the phases must not leak into each other).
BB_DEV void ring_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

struct PingState {
  bf16x8_t qf[PD / 16];
  f32x16_t o[PD / 32];
  f32x16_t s[2];       // S^T of the current tile, per 32-key half
  bf16x8_t pk[2][2];   // P^T fragments of the previous tile
  float m, l;
};

// S(t) = K Q^T (16 MFMAs).
template <bool F16>
BB_DEV void ping_qk(PingState& st, const uint16_t* kl, int li, int h) {
  st.s[0] = f32x16_t{};
  st.s[1] = f32x16_t{};
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int dk = 0; dk < PD / 16; ++dk) {
      const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(kl + k_off<PD>(32 * kb + li, 2 * dk + h)));
      st.s[kb] = mma32<F16>(a, st.qf[dk], st.s[kb]);
    }
}

// O^T += V^T P^T (16 MFMAs).
template <bool F16>
BB_DEV void ping_pv(PingState& st, const uint16_t* vt, int li, int h) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int unit = 2 * (2 * kb + u) + h;
#pragma unroll
      for (int dv = 0; dv < PD / 32; ++dv) {
        const int d = 32 * dv + li;
        st.o[dv] = mma32<F16>(as_bf16x8(*reinterpret_cast<const u32x4_t*>(vt + vt_off(d, unit))), st.pk[kb][u], st.o[dv]);
      }
    }
}

// MFMA phase of the window loop: O^T += V^T(t-1) P(t-1)^T (16 MFMAs), then S(t) = K(t) Q^T (16 MFMAs), with the LDS
// fragment reads software-pipelined four MFMAs ahead through a register ring (the LDS latency would otherwise idle the
// matrix core between each read and the MFMA that consumes it). Fragment i < 16 is the V^T fragment of PV step
// (kb, u, dv) = (i / 8, i / 4 % 2, i % 4); fragment 16 + j the K fragment of QK step (kb, dk) = (j % 2, j / 2): the
// two key halves' chains interleave, so consecutive MFMAs share their Q operand (each chain still sums dk in order).
constexpr int kRing = 4;

// Per-lane byte offsets of the fragments inside a K tile (k[dk], key half 0; half 1 is 8192 bytes on) and a V^T tile
// (v[2 a + u] for d block 0; d block dv is 4096 dv bytes on, with a = kb ^ (dv & 1), since vt_swz(32 dv + li) =
// vt_swz(li) ^ 4 (dv & 1)). With them a fragment address is one add of the tile's wave-uniform LDS address plus an
// immediate.
struct FragOfs {
  uint32_t k[PD / 16];
  uint32_t v[4];
};
BB_DEV FragOfs frag_ofs(int li, int h) {
  FragOfs f;
#pragma unroll
  for (int dk = 0; dk < PD / 16; ++dk) f.k[dk] = 2u * (uint32_t)k_off<PD>(li, 2 * dk + h);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int u = 0; u < 2; ++u) f.v[2 * a + u] = 2u * (uint32_t)vt_off(li, 4 * a + 2 * u + h);
  return f;
}
BB_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(
      reinterpret_cast<__attribute__((address_space(3))) const void*>(reinterpret_cast<uintptr_t>(p)));
}
BB_DEV u32x4_t lds16(uint32_t addr) {
  return *(const __attribute__((address_space(3))) u32x4_t*)(uintptr_t)addr;
}
// The tile's fragment base addresses, one add each, kept opaque so that the per-fragment constants go into the
// ds_read offset field instead of being folded into the scalar and added per read.
struct FragBase {
  uint32_t k[PD / 16];
  uint32_t v[4];
};
BB_DEV FragBase frag_base(uint32_t kl, uint32_t vt, const FragOfs& f) {
  FragBase b;
#pragma unroll
  for (int j = 0; j < PD / 16; ++j) {
    b.k[j] = kl + f.k[j];
    asm volatile("" : "+v"(b.k[j]));
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b.v[j] = vt + f.v[j];
    asm volatile("" : "+v"(b.v[j]));
  }
  return b;
}
BB_DEV u32x4_t ping_frag_at(const FragBase& b, int i) {
  if (i < 16) {
    const int kb = i / 8, u = (i / 4) % 2, dv = i % 4;
    return lds16(b.v[2 * (kb ^ (dv & 1)) + u] + 4096u * dv);
  }
  const int j = i - 16, kb = j % 2, dk = j / 2;
  return lds16(b.k[dk] + 8192u * kb);
}

template <bool F16>
BB_DEV void ping_mfma_phase(PingState& st, uint32_t kl, uint32_t vt, const FragOfs& fo) {
  const FragBase fb = frag_base(kl, vt, fo);
  u32x4_t ring[kRing];
#pragma unroll
  for (int i = 0; i < kRing; ++i) ring[i] = ping_frag_at(fb, i);
  st.s[0] = f32x16_t{};
  st.s[1] = f32x16_t{};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const bf16x8_t a = as_bf16x8(ring[i % kRing]);
    if (i < 16) {
      const int kb = i / 8, u = (i / 4) % 2, dv = i % 4;
      st.o[dv] = mma32<F16>(a, st.pk[kb][u], st.o[dv]);
    } else {
      const int j = i - 16, kb = j % 2, dk = j / 2;
      st.s[kb] = mma32<F16>(a, st.qf[dk], st.s[kb]);
    }
    if (i + kRing < 32) ring[i % kRing] = ping_frag_at(fb, i + kRing);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// P(t) = 2^(S(t) c - m) as bf16 MFMA fragments; returns this lane's sum of the fp32 values.
template <bool F16>
BB_DEV float ping_exp(PingState& st, float c) {
  const float nm = -st.m;
  float sum = 0.0f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float pe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pe[e] = fast_exp2(fmaf(st.s[kb][8 * u + e], c, nm));
        sum = kb == 0 && u == 0 && e == 0 ? pe[e] : sum + pe[e];  // no 0 + p[0] add
      }
      st.pk[kb][u] = as_bf16x8(u32x4_t{pack2<F16>(pe[0], pe[1]), pack2<F16>(pe[2], pe[3]),
                                       pack2<F16>(pe[4], pe[5]), pack2<F16>(pe[6], pe[7])});
    }
  return sum;
}

// Tile maximum of S(t) over the 64 keys of this lane's query, times c.
BB_DEV float ping_tile_max(const PingState& st, float c) {
  // NaN-propagating maximum (v_maximum3_f32): fmaxf would first canonicalise every MFMA result
  float mx = __builtin_elementwise_maximum(st.s[0][0], st.s[1][0]);
#pragma unroll
  for (int r = 1; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(st.s[0][r], st.s[1][r]));
  return xhalf_max(mx) * c;
}

// Moves the exponent offset of the lanes with `need` to mt, rescaling O and l.
BB_DEV void ping_rescale(PingState& st, bool need, float mt) {
  const float alpha = need ? fast_exp2(st.m - mt) : 1.0f;
  if (need) st.m = mt;
  st.l *= alpha;
#pragma unroll
  for (int dv = 0; dv < PD / 32; ++dv)
#pragma unroll
    for (int r = 0; r < 16; ++r) st.o[dv][r] *= alpha;
}

// Online softmax of a masked tile S(t) into P(t): running offset m (log2 units), sum l, O rescaled when the tile
// maximum exceeds m by more than kRescaleThreshold.
template <bool F16, typename Mask>
BB_DEV void ping_softmax_masked(PingState& st, float c, int64_t q, const Mask& mask, int h) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const uint32_t bits = mask.bits(q, kb, h);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (!((bits >> r) & 1u)) st.s[kb][r] = -__builtin_huge_valf();
  }
  const float mt = ping_tile_max(st, c);
  const bool need = mt > st.m + kRescaleThreshold;
  if (__builtin_amdgcn_ballot_w64(need)) ping_rescale(st, need, mt);
  st.l += ping_exp<F16>(st, c);
}

// Online softmax of a tile with no masked element. The tile is exponentiated against the current offset first;
// only when a probability may exceed 2^kRescaleThreshold (this lane's or the partner lane's sum does: every term is
// at most the sum; an infinite or NaN sum counts too) is the tile maximum taken, the offset moved and the tile
// exponentiated again. Same bound on P as the masked form, without a maximum per tile in the common case.
template <bool F16>
BB_DEV void ping_softmax_open(PingState& st, float c) {
  float sum = ping_exp<F16>(st, c);
  const float lim = __builtin_amdgcn_exp2f(kRescaleThreshold);
  const bool over = !(sum <= lim);
  if (__builtin_amdgcn_ballot_w64(over)) {  // some lane needs it, so some row does: only then pair up the lanes
    const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)over, (uint32_t)over, false, false);
    const bool need = (sw[0] | sw[1]) != 0u;
    const float mt = ping_tile_max(st, c);
    // the new offset never goes below the old one, so rows that do not need it keep theirs
    ping_rescale(st, need, __builtin_elementwise_maximum(mt, st.m));
    sum = ping_exp<F16>(st, c);
  }
  st.l += sum;
}

// Work item of a workgroup and the rows of one wave: (KV head, row tile of 32 x 8 / HPW rows, key chunk), XCD-aware as
// in flash_kernel.
struct PipeItem {
  int bh, kvbh, chunk;
  int64_t T_eff, r1, qlo, qhi, rw, qw0, qw1, qme;
  bool wave_live;
};

template <int HPW>
BB_DEV PipeItem pipe_item(const FlashParams& p, int bid, int hd, int rbk, int li) {
  constexpr int PROWS = 32 * (PNW / HPW);
  const int lanes_total = p.n_kvbh * p.head_splits;
  const int per_lane = p.row_tiles * p.n_chunks;  // split mode: (row tile, key chunk) pairs
  int lane_id, within;
  if (p.remap) {
    const int x = bid & 7, sidx = bid >> 3;
    lane_id = x + 8 * (sidx / per_lane);
    within = sidx % per_lane;
  } else {
    lane_id = bid % lanes_total;
    within = bid / lanes_total;
  }
  PipeItem it;
  const int rt = p.row_tiles - 1 - within / p.n_chunks;
  it.chunk = within % p.n_chunks;
  it.kvbh = lane_id / p.head_splits;
  const int hsplit = lane_id % p.head_splits;
  const int batch = it.kvbh / p.Hkv_pb;
  it.bh = batch * p.H + (it.kvbh % p.Hkv_pb) * p.G + hsplit * HPW + hd;
  it.T_eff = p.row_end < p.T ? p.row_end : p.T;
  const int64_t r0 = (int64_t)rt * PROWS;
  it.r1 = (r0 + PROWS < it.T_eff ? r0 + PROWS : it.T_eff) - 1;
  it.qlo = p.offset + r0 * p.pos_step;
  it.qhi = p.offset + it.r1 * p.pos_step;
  it.rw = r0 + 32 * rbk;  // first row of this wave
  it.wave_live = it.rw <= it.r1;
  it.qw0 = p.offset + it.rw * p.pos_step;
  it.qw1 = p.offset + (it.rw + 31 < it.r1 ? it.rw + 31 : it.r1) * p.pos_step;
  it.qme = it.qw0 + li * p.pos_step;  // this lane's query position
  return it;
}

// GATHER: the routed phase gathers the rows of its batches itself (route lists with several groups, where no tiles
// are pre-gathered); a separate instantiation, so that the common kernel's register allocation is not affected.
// HPW: query heads per workgroup (4 when a KV head serves a multiple of 4 query heads; 2 and 1 for 2 and 1, with
// 4 and 8 row blocks of 32 rows), so every staged K / V^T tile is read by all 8 waves in each case.
template <bool F16, bool GATHER, int HPW>
__global__ __launch_bounds__(64 * PNW, 1) void flash_ping_kernel(FlashParams p) {
  static_assert(HPW == 4 || HPW == 2 || HPW == 1, "4, 2 or 1 query heads per workgroup");
  constexpr int RB = PNW / HPW;  // row blocks (waves) per head
  __shared__ __attribute__((aligned(1024))) uint16_t smem[PLDS];
  __shared__ __attribute__((aligned(16))) int32_t route_keys[HPW][kRouteCache];
  __shared__ int head_batches[RB][HPW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, li = lane & 31;
  const int hd = wave % HPW, rbk = wave / HPW;  // head slot, row block
  const int grp = wave >> 2;                    // ping-pong group: waves w and w + 4 share a SIMD

  // ---- work item: (KV head, row tile), XCD-aware as in flash_kernel ----
  PipeItem it = pipe_item<HPW>(p, blockIdx.x, hd, rbk, li);
  const int bh = it.bh, kvbh = it.kvbh, chunk = it.chunk;
  const int64_t T_eff = it.T_eff, r1 = it.r1, qlo = it.qlo, qhi = it.qhi, rw = it.rw;
  const bool wave_live = it.wave_live;
  const int64_t qw0 = it.qw0, qw1 = it.qw1, qme = it.qme;

  PingState st;
  {
    const int64_t row = rw + li;
    const bool live = row < T_eff;
    const uint16_t* qrow = p.q + (int64_t)bh * p.sq0 + (live ? row : T_eff - 1) * p.sq1 + 8 * h;
#pragma unroll
    for (int dk = 0; dk < PD / 16; ++dk) {
      const u32x4_t v = ld16(qrow + 16 * dk);
      st.qf[dk] = as_bf16x8(live ? v : u32x4_t{0, 0, 0, 0});
    }
#pragma unroll
    for (int dv = 0; dv < PD / 32; ++dv) st.o[dv] = f32x16_t{};
    st.m = -1.0e20f;
    st.l = 0.0f;
  }

  const uint16_t* kbase = p.k + (int64_t)kvbh * p.sk0;
  const uint16_t* vbase = p.v + (int64_t)kvbh * p.sv0;
  const uint16_t* vtbase = p.vt + (int64_t)kvbh * PD * p.np;

  // ---- tiles (64-aligned): front range [0, f1) and window range [w0, w1) ----
  const int64_t front_end = p.front < qhi + 1 ? p.front : qhi + 1;
  int64_t wlo = qlo - p.window + 1;
  if (wlo < 0) wlo = 0;
  int64_t f1 = front_end > 0 ? (front_end + kTileKeys - 1) / kTileKeys : 0;
  int64_t w0 = wlo / kTileKeys;
  const int64_t w1 = qhi / kTileKeys + 1;
  if (w0 <= f1) {  // the ranges touch: one range from 0
    f1 = 0;
    w0 = 0;
  }
  // Tiles every row of the workgroup attends in full: j with 64j+63 <= qlo and (64j+63 < front or
  // 64j >= qhi - window + 1), i.e. [0, ua) from the front and [ub, uc) in the window. They run through the ping-pong
  // loop with no element mask; the few edge tiles (window start, diagonal, a partial front tile) follow.
  const int64_t a_lim = (p.front < qlo + 1 ? p.front : qlo + 1) / kTileKeys;
  const int64_t ua = a_lim < (f1 > 0 ? f1 : w1) ? a_lim : (f1 > 0 ? f1 : w1);
  int64_t ub = qhi - p.window + 1 <= 0 ? 0 : (qhi - p.window + 1 + kTileKeys - 1) / kTileKeys;
  if (ub < w0) ub = w0;
  if (ub < ua) ub = ua;
  int64_t uc = (qlo + 1) / kTileKeys;
  if (uc > w1) uc = w1;
  if (uc < ub) uc = ub;
  // split mode (exact tail: no routes): only the tiles of key chunk `chunk`, [c0, c1)
  int64_t c0 = 0, c1 = w1 > f1 ? w1 : f1;
  if (p.n_chunks > 1) {
    c0 = (int64_t)chunk * p.key_chunk / kTileKeys;
    const int64_t ce = ((int64_t)chunk + 1) * p.key_chunk / kTileKeys;
    if (ce < c1) c1 = ce;
  }
  auto clip = [&](int64_t& a, int64_t& b) {
    if (a < c0) a = c0;
    if (b > c1) b = c1;
    if (b < a) b = a;
  };
  int64_t ua0 = 0, ua1 = ua;
  clip(ua0, ua1);
  clip(ub, uc);
  const int nu = (int)((ua1 - ua0) + (uc - ub));
  // The remaining tiles of [0, f1) u [w0, w1) need element masks: front tiles past the unmasked prefix [ua1, f1),
  // the window start [max(w0, ua1), ub) and the diagonal [uc, w1) (typically one tile each for the last two). They
  // run in the same loop, after the unmasked ones, with the masked softmax.
  int64_t ma0 = ua1, ma1 = f1 > 0 ? f1 : ua1;
  int64_t mb0 = w0 > ua1 ? w0 : ua1, mb1 = ub;
  int64_t mc0 = uc, mc1 = w1;
  clip(ma0, ma1);
  clip(mb0, mb1);
  clip(mc0, mc1);
  const int ntot = nu + (int)((ma1 - ma0) + (mb1 - mb0) + (mc1 - mc0));
  // tile of list entry t: t + the offset of the range t falls in, as a sum of 32-bit steps (scalar selects; kept
  // wave-uniform explicitly so that the buffer loads take it as a scalar offset)
  const int n1 = (int)(ua1 - ua0), n2 = nu, n3 = n2 + (int)(ma1 - ma0), n4 = n3 + (int)(mb1 - mb0);
  const int d1 = (int)ua0, e2 = (int)ub - n1 - d1, e3 = (int)(ma0 - ub) - (n2 - n1), e4 = (int)(mb0 - ma0) - (n3 - n2),
            e5 = (int)(mc0 - mb0) - (n4 - n3);
  auto upos = [=](int t) -> int64_t {
    const int d = d1 + (t >= n1 ? e2 : 0) + (t >= n2 ? e3 : 0) + (t >= n3 ? e4 : 0) + (t >= n4 ? e5 : 0);
    return (int64_t)__builtin_amdgcn_readfirstlane(t + d) * kTileKeys;
  };
  // VALU phase of tile t: the lazy softmax for unmasked tiles, the masked one (front | causal window) otherwise
  auto softmax_masked = [&](int t) {
    const int64_t k0 = upos(t), k1 = k0 + kTileKeys - 1;
    const bool live = wave_live && k0 <= qw1 && !(k0 >= p.front && k1 <= qw0 - p.window);
    ping_softmax_masked<F16>(st, p.c, qme, PipeWindowMask{k0, p.front, p.window, live}, h);
  };
  auto softmax = [&](int t) {
    if (t < nu) ping_softmax_open<F16>(st, p.c);
    else softmax_masked(t);
  };

  uint16_t* ring = smem;
  auto kst = [&](int t) { return ring + (t & (PST - 1)) * 2 * PTE; };
  auto vst = [&](int t) { return ring + (t & (PST - 1)) * 2 * PTE + PTE; };
  const FragOfs fo = frag_ofs(li, h);
  TileLoader ld;
  ld.init(kbase, p.sk1, p.N, vtbase, p.np, wave, lane);

  if (ntot > 0) {
    ld.tile(kst(0), vst(0), upos(0));
    if (ntot > 1) ld.tile(kst(1), vst(1), upos(1));
    vm_wait_tile(ntot > 1);
    ring_barrier();
    if (grp == 1) ring_barrier();  // waves 4..7 run one phase behind
    // tile 0: QK only
    if (ntot > 2) ld.tile(kst(2), vst(2), upos(2));
    ping_qk<F16>(st, kst(0), li, h);
    vm_wait_tile(ntot > 2);
    ring_barrier();
    softmax(0);
    ring_barrier();
    // Two copies of the loop body, unmasked tiles then masked ones, so that the register allocation of the hot one
    // does not carry the mask arithmetic.
    for (int t = 1; t < nu; ++t) {
      // MFMA phase: PV of tile t-1, QK of tile t
      __builtin_amdgcn_s_setprio(1);
      ping_mfma_phase<F16>(st, lds_addr(kst(t)), lds_addr(vst(t - 1)), fo);
      __builtin_amdgcn_s_setprio(0);
      vm_wait_tile(false);  // tile t+1 has landed
      ring_barrier();
      // VALU phase: softmax of tile t, then tile t+2 starts loading into the stage tile t-2 used (every wave is past
      // the MFMA phase that last read it). The loads come after the exponentials: issuing a direct load stalls the
      // wave for as long as the CU's address unit is busy with the other waves' loads.
      ping_softmax_open<F16>(st, p.c);
      if (t + 2 < ntot) ld.tile(kst(t + 2), vst(t + 2), upos(t + 2));
      ring_barrier();
    }
    // every tile of this loop is masked: t >= max(nu, 1) >= nu
#pragma unroll 1
    for (int t = nu > 1 ? nu : 1; t < ntot; ++t) {
      __builtin_amdgcn_s_setprio(1);
      ping_mfma_phase<F16>(st, lds_addr(kst(t)), lds_addr(vst(t - 1)), fo);
      __builtin_amdgcn_s_setprio(0);
      vm_wait_tile(false);
      ring_barrier();
      softmax_masked(t);
      if (t + 2 < ntot) ld.tile(kst(t + 2), vst(t + 2), upos(t + 2));
      ring_barrier();
    }
    ping_pv<F16>(st, vst(ntot - 1), li, h);
    if (grp == 0) ring_barrier();  // realign the two groups
  }

  // The work item again, from copies of the block and lane indices that the compiler cannot see through: the values
  // the routed phase and the epilogue need are recomputed here instead of being held (and spilled) across the loop.
  {
    int bid2 = blockIdx.x, li2 = li;
    asm volatile("" : "+s"(bid2));
    asm volatile("" : "+v"(li2));
    it = pipe_item<HPW>(p, bid2, hd, rbk, li2);
  }
  // ---- routed keys: per-head tiles pre-gathered by route_tiles_kernel; the RB waves of a head share the loads ----
  if (p.route_k > 0) {
    __syncthreads();  // every wave is done with the ring
    uint16_t* kl = smem + hd * 2 * PTE;
    uint16_t* vt = kl + PTE;
    int64_t g_first = it.qlo / p.route_chunk, g_last = it.qhi / p.route_chunk;
    if (g_last >= p.n_groups) g_last = p.n_groups - 1;
    const uint32_t loff = 16u * (uint32_t)lane;
    for (int64_t g = g_first; g <= g_last; ++g) {
      const int32_t* irow = p.idx + (int64_t)it.bh * p.si0 + g * p.si1;
      // This head's pre-gathered batches of group g: batch b is a K tile at b * 2 PTE and its V^T tile after it.
      // Each of the head's RB waves loads blocks rbk + RB i (i < 16 / RB) of a tile straight into LDS.
      const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(p.rtiles + ((int64_t)it.bh * p.n_groups + g) * p.rt_batches * 2 * PTE), 0,
          p.rt_batches * 2 * PTE * 2, 0x00020000);
      auto load_tile = [&](int b, uint16_t* dst, int part) {
#pragma unroll
        for (int i = 0; i < PBLK / RB; ++i) {
          const int blk = rbk + RB * i;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rrs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                       reinterpret_cast<uintptr_t>(dst + blk * 512)),
              16, loff, (b * 2 * PTE + part * PTE + blk * 512) * 2, 0, 0);
        }
      };
      // The head's route slots, kRouteCache at a time, go to LDS in one pass (usable keys, -1 elsewhere: a key some
      // row of the workgroup attends is >= front, < N and <= it.qhi - window). Batches of 64 slots run up to the last
      // one holding a usable key.
      for (int sb = 0; sb < p.route_k; sb += kRouteCache) {
        const int nslots = p.route_k - sb < kRouteCache ? p.route_k - sb : kRouteCache;
        int nbh = 0;
        for (int s0 = 64 * rbk; s0 < kRouteCache; s0 += 64 * RB) {
          const int sl = s0 + lane;
          const int64_t key = sl < nslots ? irow[(int64_t)(sb + sl) * p.si2] : -1;
          const bool ok = key >= p.front && key < p.N && key <= it.qhi - p.window;
          route_keys[hd][sl] = ok ? (int32_t)key : -1;
          if (__builtin_amdgcn_ballot_w64(ok)) nbh = s0 / kTileKeys + 1;
        }
        if (lane == 0) head_batches[rbk][hd] = nbh;  // each of the head's RB waves scanned 1 / RB of the slots
        __syncthreads();
        int nb = 0, my_nb = 0;
#pragma unroll
        for (int x = 0; x < HPW; ++x)
#pragma unroll
          for (int y = 0; y < RB; ++y) {
            const int v = head_batches[y][x];
            nb = nb > v ? nb : v;
            if (x == hd) my_nb = my_nb > v ? my_nb : v;
          }
        __syncthreads();  // head_batches and route_keys are rewritten only after every wave has read them
        const int b0 = sb / kTileKeys;
        for (int bi = 0; bi < nb; ++bi) {
          const bool work = bi < my_nb;
          const int32_t* keys = route_keys[hd] + kTileKeys * bi;
          if constexpr (!GATHER) {
            if (work) {
              load_tile(b0 + bi, kl, 0);
              load_tile(b0 + bi, vt, 1);
            }
          } else if (work) {
            // No pre-gathered tiles (several route groups): the head's waves gather the batch's rows here. K rows
            // go straight to LDS (empty slots read row 0, masked out); V rows are transposed through registers in
            // units of 4 keys x 8 d into the permuted V^T layout. Only batches holding a usable key are gathered.
            const uint16_t* kb = p.k + (int64_t)it.kvbh * p.sk0;
            const uint16_t* vb = p.v + (int64_t)it.kvbh * p.sv0;
            for (int b = rbk; b < PBLK; b += RB) {
              const int e = b * 512 + 8 * lane;
              const int row = e / PD, chk = ((e % PD) / 8) ^ (row & (PD / 8 - 1));
              const int32_t kr = keys[row];
              lds_dma16(kb + (int64_t)(kr >= 0 ? kr : 0) * p.sk1 + 8 * chk, kl + b * 512);
            }
            for (int u = lane + 64 * rbk; u < (kTileKeys / 4) * (PD / 8); u += 64 * RB) {
              const int bq = u % (PD / 8), a4 = u / (PD / 8);
              u32x4_t vr[4];
#pragma unroll
              for (int s2 = 0; s2 < 4; ++s2) {
                const int32_t kr = keys[4 * a4 + s2];
                vr[s2] = kr >= 0 ? ld16(vb + (int64_t)kr * p.sv1 + 8 * bq) : u32x4_t{0, 0, 0, 0};
              }
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t lo = __builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel);
                const uint32_t hi = __builtin_amdgcn_perm(vr[3][e >> 1], vr[2][e >> 1], sel);
                *reinterpret_cast<u32x2_t*>(vt + vt_off(8 * bq + e, 2 * (a4 >> 2) + (a4 & 1)) + 4 * ((a4 >> 1) & 1)) =
                    u32x2_t{lo, hi};
              }
            }
          }
          vm_wait_tile(false);
          __syncthreads();
          if (work && it.wave_live) {
            const PipeRoutedMask rm{keys, p.window, p.route_chunk, g};
            ping_qk<F16>(st, kl, li, h);
            ping_softmax_masked<F16>(st, p.c, it.qme, rm, h);
            ping_pv<F16>(st, vt, li, h);
          }
          __syncthreads();
        }
      }
    }
  }

  // ---- epilogue ----
  if (p.route_k <= 0) __syncthreads();  // the ring is free for the output staging (the routed phase ends on one)
  if (!it.wave_live) return;
  const float lt = xhalf_sum(st.l);
  if (p.n_chunks > 1) {  // partial (O, m, l) of this key chunk for flash_merge_kernel
    // The fp32 rows pass through this wave's 16 KB of LDS (row r at r * 512 bytes, its 16-byte chunk k in slot
    // k ^ (r % 16)) so that every global store writes two whole rows, as for the output below.
    float* fstage = reinterpret_cast<float*>(smem) + wave * (32 * PD);
#pragma unroll
    for (int dv = 0; dv < PD / 32; ++dv)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int k = 8 * dv + 2 * g4 + h;
        *reinterpret_cast<f32x4_t*>(fstage + li * PD + 4 * (k ^ (li & 15))) =
            f32x4_t{st.o[dv][4 * g4], st.o[dv][4 * g4 + 1], st.o[dv][4 * g4 + 2], st.o[dv][4 * g4 + 3]};
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t base0 = ((int64_t)it.chunk * p.BH + it.bh) * p.T + it.rw;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 2 * i + (lane >> 5), k = lane & 31;
      const f32x4_t v = *reinterpret_cast<const f32x4_t*>(fstage + r * PD + 4 * (k ^ (r & 15)));
      if (it.rw + r < it.T_eff) *reinterpret_cast<f32x4_t*>(p.part_o + (base0 + r) * PD + 4 * k) = v;
    }
    const int64_t row = it.rw + li;
    if (h == 0 && row < it.T_eff) {
      p.part_ml[2 * (base0 + li)] = st.m;
      p.part_ml[2 * (base0 + li) + 1] = lt;
    }
    return;
  }
  // The normalised rows pass through this wave's 8 KB of LDS (row r at r * 256 bytes, its 16-byte chunk k in slot
  // k ^ (r % 16)), so that every global store writes two whole rows: lane l of store i takes bytes 8 (l % 32) .. of
  // row 2 i + l / 32. Stored from the fragment layout, each store would touch 32 rows.
  const float inv = 1.0f / fmaxf(lt, 1.0e-20f);
  uint16_t* stage = smem + wave * (32 * PD);
#pragma unroll
  for (int dv = 0; dv < PD / 32; ++dv)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int k = 4 * dv + g4;
      const u32x2_t w = {pack2<F16>(st.o[dv][4 * g4] * inv, st.o[dv][4 * g4 + 1] * inv),
                         pack2<F16>(st.o[dv][4 * g4 + 2] * inv, st.o[dv][4 * g4 + 3] * inv)};
      *reinterpret_cast<u32x2_t*>(stage + li * PD + 8 * (k ^ (li & 15)) + 4 * h) = w;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint16_t* obase = p.out + (int64_t)it.bh * p.so0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 2 * i + (lane >> 5), q = lane & 31, k = q >> 1;
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(stage + r * PD + 8 * (k ^ (r & 15)) + 4 * (q & 1));
    const int64_t row = it.rw + r;
    if (row < it.T_eff) *reinterpret_cast<u32x2_t*>(obase + row * p.so1 + 4 * q) = w;
  }
}

// Pre-gathers, per query head and route group, the routed K rows and V^T columns of every 64-slot batch into the
// LDS tile layouts of the main pass (K tile: row r, 16-byte chunk c at r * D + 8 (c ^ (r % 16)); V^T tile: vt_off),
// so that the routed phase streams them with direct loads like window tiles. Empty slots (-1, or outside [0, N))
// are zero rows. Grid (batches, n_groups, BH), 256 threads.
__global__ __launch_bounds__(256) void route_tiles_kernel(FlashParams p, uint16_t* __restrict__ rt) {
  const int b = blockIdx.x, g = blockIdx.y, bh = blockIdx.z, t = threadIdx.x;
  const int batch = bh / p.H;
  const int kvbh = batch * p.Hkv_pb + (bh % p.H) / p.G;
  const uint16_t* kbase = p.k + (int64_t)kvbh * p.sk0;
  const uint16_t* vbase = p.v + (int64_t)kvbh * p.sv0;
  const int32_t* irow = p.idx + (int64_t)bh * p.si0 + (int64_t)g * p.si1;
  uint16_t* kt = rt + (((int64_t)bh * p.n_groups + g) * p.rt_batches + b) * 2 * PTE;
  uint16_t* vtt = kt + PTE;
  auto key_of = [&](int r) -> int64_t {
    const int slot = b * kTileKeys + r;
    const int64_t key = slot < p.route_k ? irow[(int64_t)slot * p.si2] : -1;
    return key >= 0 && key < p.N ? key : -1;
  };
  // K tile: 64 rows x 16 chunks of 16 bytes, 4 per thread
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = t + 256 * i, row = u / 16, chunk = u % 16;
    const int64_t key = key_of(row);
    const u32x4_t v = key >= 0 ? ld16(kbase + key * p.sk1 + 8 * chunk) : u32x4_t{0, 0, 0, 0};
    st16(kt + row * PD + 8 * (chunk ^ (row & 15)), v);
  }
  // V^T tile: unit (4 keys x 8 d) per thread, transposed into the permuted key order of vt_off
  const int bq = t % (PD / 8), a4 = t / (PD / 8);
  u32x4_t vr[4];
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
    const int64_t key = key_of(4 * a4 + s2);
    vr[s2] = key >= 0 ? ld16(vbase + key * p.sv1 + 8 * bq) : u32x4_t{0, 0, 0, 0};
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int w = e >> 1;
    const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
    const uint32_t lo = __builtin_amdgcn_perm(vr[1][w], vr[0][w], sel);
    const uint32_t hi = __builtin_amdgcn_perm(vr[3][w], vr[2][w], sel);
    const int d = 8 * bq + e;
    *reinterpret_cast<u32x2_t*>(vtt + vt_off(d, 2 * (a4 >> 2) + (a4 & 1)) + 4 * ((a4 >> 1) & 1)) = u32x2_t{lo, hi};
  }
}

}  // namespace

bool flash_pipe_supported(const FlashParams& p, int D, int hpw) {
  // Buffer offsets are unsigned 32-bit: every K offset up to the end of the last tile (row N + 63, which reads as
  // zero) and every V^T offset of one KV head must stay below 4 GiB, so that no offset wraps back into the
  // tensor. Split mode needs whole tiles.
  const int64_t lim = (int64_t)1 << 32;
  const bool fits = (p.N + kTileKeys) * p.sk1 * 2 < lim && (int64_t)PD * p.np * 2 < lim;
  const bool chunks_ok = p.n_chunks == 1 || (p.key_chunk % kTileKeys == 0 && p.route_k == 0);
  // 4, 2 or 1 query heads per workgroup; the in-kernel gather of several route groups is built for 4
  const bool heads_ok = (hpw == 4 || hpw == 2 || hpw == 1) && p.G % hpw == 0 &&
                        (hpw == 4 || p.route_k == 0 || p.n_groups == 1);
  return D == PD && heads_ok && p.key_mask == nullptr && fits && chunks_ok;
}

size_t route_tiles_bytes(int BH, int n_groups, int route_k) {
  if (BH <= 0 || n_groups <= 0 || route_k <= 0) return 0;
  return (size_t)BH * n_groups * ((route_k + kTileKeys - 1) / kTileKeys) * 2 * PTE * sizeof(uint16_t);
}

hipError_t launch_route_tiles(const FlashParams& p, uint16_t* rt, hipStream_t stream) {
  if (p.route_k <= 0) return hipSuccess;
  hipLaunchKernelGGL(route_tiles_kernel, dim3((unsigned)p.rt_batches, (unsigned)p.n_groups, (unsigned)p.BH), dim3(256),
                     0, stream, p, rt);
  return hipGetLastError();
}

hipError_t launch_flash_pipe(const FlashParams& p, int hpw, hipStream_t stream) {
  const int64_t items = (int64_t)p.n_kvbh * p.head_splits * p.row_tiles * p.n_chunks;
  if (items <= 0) return hipSuccess;
  if (items > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)items), block(64 * PNW);
  const bool gather = p.route_k > 0 && !p.rtiles;
  if (gather && hpw != 4) return hipErrorInvalidValue;
  if (gather) {
    if (p.f16) hipLaunchKernelGGL((flash_ping_kernel<true, true, 4>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_ping_kernel<false, true, 4>), grid, block, 0, stream, p);
  } else if (hpw == 4) {
    if (p.f16) hipLaunchKernelGGL((flash_ping_kernel<true, false, 4>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_ping_kernel<false, false, 4>), grid, block, 0, stream, p);
  } else if (hpw == 2) {
    if (p.f16) hipLaunchKernelGGL((flash_ping_kernel<true, false, 2>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_ping_kernel<false, false, 2>), grid, block, 0, stream, p);
  } else if (hpw == 1) {
    if (p.f16) hipLaunchKernelGGL((flash_ping_kernel<true, false, 1>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((flash_ping_kernel<false, false, 1>), grid, block, 0, stream, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace bb
