// Ping-pong sink + causal window + routed sparse flash attention for gfx950 (head_dim 128, no token mask): the main
// pass of Bigger Bird v3 prefill at production shape.
//
// Same semantics as bb_flash.hip (kernels/bigger_bird_flash.py:42-96 of the reference). Work decomposition:
//   * a workgroup = 8 waves = the 4 query heads of one KV head x 2 blocks of 32 query rows (64 rows); every K / V^T
//     tile staged in LDS is read by all 8 waves (GQA reuse inside the workgroup). With 2 query heads per KV head a
//     workgroup is 2 heads x 4 row blocks (128 rows), with 1 (MHA) one head x 8 row blocks (256 rows), so the tiles
//     are still shared by all 8 waves;
//   * the matrix products run on v_mfma_f32_16x16x32 (bf16 or fp16). A wave's 32 query rows are two blocks of 16, and
//     every K or V^T fragment read from LDS feeds the MFMAs of both blocks: the same LDS bytes per FLOP as a 32x32x16
//     layout, with a quarter of the accumulator registers per instruction. On random operands the part runs power-
//     limited, and the ping-pong loop below runs about 10% more FLOP/s in this shape than in the 32x32x16 one;
//   * waves w and w + 4 share a SIMD. Per 64-key tile a wave runs an MFMA phase  (O^T += V^T(t-1) P(t-1)^T,
//     S(t) = K(t) Q^T: 64 MFMAs on 32 LDS fragments) and a VALU phase (online softmax of S(t) into P(t)), separated by
//     workgroup barriers. Waves 4..7 start one barrier late, so on every SIMD one wave is in its MFMA phase while the
//     other is in its VALU phase: the matrix cores and the VALUs work at the same time instead of in turn;
//   * K and V^T tiles stream global->LDS with 16-byte buffer loads straight into LDS (no staging registers) through a
//     four-stage ring, issued two tiles ahead at the end of a VALU phase; rows past N read as zeros through the buffer
//     resource bounds;
//   * the exponent offset moves only when a probability would exceed 2^8 (O rescales stay rare); tiles without masked
//     elements skip the per-tile maximum unless the row sum says the offset must move;
//   * routed keys differ per head: after the window loop the waves of a head stream its routed K / V^T tiles into
//     that head's LDS tile, pre-gathered per 64-slot batch by route_tiles_kernel (one route group), or gather the
//     batch's K rows and V rows themselves (several route groups: the GATHER instantiation).
//
// Register layouts (lane l = x + 16 a, x = l % 16, a = l / 16; a wave's row r = 16 rb + x, rb = 0, 1):
//   * 16x16x32 MFMA: A[m][k] at lane m + 16 (k / 8), element k % 8; B[k][n] at lane n + 16 (k / 8), element k % 8;
//     D[m][n] at lane n + 16 (m / 4), element m % 4;
//   * S^T = K Q^T per key block kb (16 keys) and row block rb: element i of lane l is key kmap(kb, 4 a + i) of row
//     16 rb + x, with kmap(kb, m) = 32 (kb / 2) + 8 (kb % 2) + 16 (m / 8) + (m % 8): blocks 0 and 2 hold keys
//     {0-7, 16-23} of their 32-key step, blocks 1 and 3 keys {8-15, 24-31};
//   * P^T for PV step st (keys 32 st ..): lane l holds row 16 rb + x, elements j < 4 from S^T block 2 st and j >= 4
//     from block 2 st + 1, element i: keys 32 st + 16 (a / 2) + 4 (a % 2) + {i, 8 + i}. That is unit 4 st + a of the
//     global V^T layout (its 16-key groups store keys 0-3, 8-11, 4-7, 12-15), so each V^T fragment is one 16-byte
//     unit per lane;
//   * O^T: lane l, d block db (16 rows of d), row block rb: element i is d = 16 db + 4 a + i of row 16 rb + x.
// A query row's 64 keys of a tile are spread over the four lanes x, x + 16, x + 32, x + 48 (16 each): the row max and
// row sum take a permlane16 and a permlane32 swap.
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

// LDS tile layouts of this kernel.
// K tile: key row r (0..63), 16-byte chunk c (d = 8c..8c+7) at element r * PD + 8 (c ^ pk_swz(r)). The 16 keys an MFMA
// key block reads at one d chunk ({0-7, 16-23} + 8 (kb % 2) + 32 (kb / 2)) sit in 16 distinct slots, and pk_swz does
// not change when a row moves by 8 (within those sets) or by 32, so a lane's fragment offsets are fixed per d chunk.
BB_DEV int pk_swz(int r) { return (r & 7) | ((r >> 1) & 8); }
BB_DEV int pk_off(int r, int c) { return r * PD + 8 * (c ^ pk_swz(r)); }
// V^T tile: row d (0..127), 8-key unit u of the global V^T layout at element d * 64 + 8 ((u + pv_rot(d)) & 7). The
// rotation depends on d % 16 only, so the d block of a fragment is an immediate offset. A ds_read_b128 serves its 64
// lanes in four 16-lane groups (measured on gfx950: lanes 32 h + 4 q + 0..3 for the quads q whose three index bits
// have the same parity), each group conflict-free when it hits 16 distinct 16-byte bank slots (address / 16 mod 16).
// This rotation leaves the fragment reads 2-way conflicting (3.2 extra LDS cycles per read, measured); the
// conflict-free rotation 2 ((d >> 1) & 3) measured 2.4% slower in the whole kernel (24.76 against 24.17 ms at 128K,
// 1.866 against 1.829 ms at 32K, interleaved A/B, identical ISA otherwise), so the conflicting one stays.
BB_DEV int pv_rot(int d) { return (d ^ ((d >> 3) & 1)) & 7; }
BB_DEV int pv_off(int d, int u) { return d * kTileKeys + 8 * ((u + pv_rot(d)) & 7); }

BB_DEV f32x4_t zero4() { return f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}; }

template <bool F16>
BB_DEV f32x4_t mma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Combining a value over the four lanes of a query row (x, x + 16, x + 32, x + 48).
BB_DEV float row4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float m = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
BB_DEV float row4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
BB_DEV bool row4_any(bool f) {
  const uint32_t v = f ? 1u : 0u;
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  const uint32_t o = a[0] | a[1];
  const auto b = __builtin_amdgcn_permlane32_swap(o, o, false, false);
  return (b[0] | b[1]) != 0u;
}

// Key offset, inside the tile, of element 0 of lane group a's S^T values in key block kb (elements i = 0..3 follow).
BB_DEV int kblk_base(int kb, int a) { return 32 * (kb >> 1) + 8 * (kb & 1) + 16 * (a >> 1) + 4 * (a & 1); }

// Bits i < n (n clamped to [0, 4]).
BB_DEV uint32_t prefix4(int64_t n) {
  const int c = (int)(n < 0 ? 0 : (n > 4 ? 4 : n));
  return (1u << c) - 1u;
}

struct PipeWindowMask {  // front | causal window (nothing when !any)
  int64_t k0, front, window;
  bool any;
  // keys k0 + kblk_base(kb, a) + i, i = 0..3, for query position q: 4 bits
  BB_DEV uint32_t bits(int64_t q, int kb, int a) const {
    if (!any) return 0u;
    const int64_t base = k0 + kblk_base(kb, a);
    const uint32_t causal = prefix4(q - base + 1);
    const uint32_t fr = prefix4(front - base);
    const uint32_t win = ~prefix4(q - window - base + 1) & 15u;
    return causal & (fr | win);
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
    // K block b = w + 8i: row 4b + lane/16, LDS slot lane%16 holds chunk (lane%16) ^ pk_swz(row); pk_swz(row) does
    // not depend on i (rows 32 apart)
    const int krow = 4 * w + lane / 16;
    kvoff = (uint32_t)krow * krow_bytes + 16u * (uint32_t)((lane % 16) ^ pk_swz(krow));
    kstep = 32u * krow_bytes;
    // V^T block b = w + 8i: d = 8b + lane/8, LDS slot lane%8 holds unit (lane%8 - pv_rot(d)) & 7; pv_rot(d) does
    // not depend on i (rows 64 apart)
    const int d = 8 * w + lane / 8;
    vvoff = (uint32_t)d * (uint32_t)(np * 2) + 16u * (uint32_t)((lane % 8 - pv_rot(d)) & 7);
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
  bf16x8_t qf[2][PD / 32];  // Q^T fragments: row block rb, d step ds (32 d each)
  f32x4_t o[PD / 16][2];    // O^T: d block db (16 d), row block rb
  f32x4_t s[4][2];          // S^T of the current tile: key block kb (16 keys), row block rb
  bf16x8_t pk[2][2];        // P^T fragments of the previous tile: 32-key step st, row block rb
  float m[2], l[2];         // per row block: exponent offset (log2 units), this lane's share of the row sum
};

// Per-lane byte offsets of the fragments inside a K tile (k[ds]: key block 0; block kb is 256 (32 (kb / 2) +
// 8 (kb % 2)) bytes on) and a V^T tile (v[st]: d block 0; d block db is 2048 db bytes on). With them a fragment
// address is one add of the tile's wave-uniform LDS address plus an immediate.
struct FragOfs {
  uint32_t k[PD / 32];
  uint32_t v[2];
};
BB_DEV FragOfs frag_ofs(int x, int a) {
  FragOfs f;
  const int r0 = 16 * (x >> 3) + (x & 7);  // key row of M-row x in key block 0
#pragma unroll
  for (int ds = 0; ds < PD / 32; ++ds) f.k[ds] = 2u * (uint32_t)pk_off(r0, 4 * ds + a);
#pragma unroll
  for (int st = 0; st < 2; ++st) f.v[st] = 2u * (uint32_t)pv_off(x, 4 * st + a);
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
  uint32_t k[PD / 32];
  uint32_t v[2];
};
BB_DEV FragBase frag_base(uint32_t kl, uint32_t vt, const FragOfs& f) {
  FragBase b;
#pragma unroll
  for (int j = 0; j < PD / 32; ++j) {
    b.k[j] = kl + f.k[j];
    asm volatile("" : "+v"(b.k[j]));
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    b.v[j] = vt + f.v[j];
    asm volatile("" : "+v"(b.v[j]));
  }
  return b;
}
// Fragment i of an MFMA phase: i < 16 the V^T fragment of PV step (st, db) = (i / 8, i % 8); 16 + j the K fragment of
// QK step (kb, ds) = (j % 4, j / 4) (consecutive K fragments belong to different key blocks, so each accumulator's
// chain over ds has three other blocks' MFMAs between its steps).
BB_DEV u32x4_t ping_frag_at(const FragBase& b, int i) {
  if (i < 16) return lds16(b.v[i / 8] + 2048u * (uint32_t)(i % 8));
  const int j = i - 16, kb = j % 4, ds = j / 4;
  return lds16(b.k[ds] + 256u * (uint32_t)(32 * (kb >> 1) + 8 * (kb & 1)));
}

template <bool F16>
BB_DEV void ping_mma(PingState& st, int i, bf16x8_t a) {
  if (i < 16) {
    const int stp = i / 8, db = i % 8;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) st.o[db][rb] = mma16<F16>(a, st.pk[stp][rb], st.o[db][rb]);
  } else {
    const int j = i - 16, kb = j % 4, ds = j / 4;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) st.s[kb][rb] = mma16<F16>(a, st.qf[rb][ds], st.s[kb][rb]);
  }
}

BB_DEV void clear_s(PingState& st) {
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) st.s[kb][rb] = zero4();
}

// S(t) = K Q^T (32 MFMAs on 16 K fragments).
template <bool F16>
BB_DEV void ping_qk(PingState& st, const uint16_t* kl, const FragOfs& fo) {
  const FragBase fb = frag_base(lds_addr(kl), 0u, fo);
  clear_s(st);
#pragma unroll
  for (int i = 16; i < 32; ++i) ping_mma<F16>(st, i, as_bf16x8(ping_frag_at(fb, i)));
}

// O^T += V^T P^T (32 MFMAs on 16 V^T fragments).
template <bool F16>
BB_DEV void ping_pv(PingState& st, const uint16_t* vt, const FragOfs& fo) {
  const FragBase fb = frag_base(0u, lds_addr(vt), fo);
#pragma unroll
  for (int i = 0; i < 16; ++i) ping_mma<F16>(st, i, as_bf16x8(ping_frag_at(fb, i)));
}

// MFMA phase of the window loop: O^T += V^T(t-1) P(t-1)^T, then S(t) = K(t) Q^T (64 MFMAs), with the 32 LDS fragment
// reads software-pipelined six fragments ahead through a register ring (the LDS latency would otherwise idle the
// matrix core between each read and the MFMAs that consume it; 4 and 8 ahead measured slower).
constexpr int kRing = 6;

template <bool F16>
BB_DEV void ping_mfma_phase(PingState& st, uint32_t kl, uint32_t vt, const FragOfs& fo) {
  const FragBase fb = frag_base(kl, vt, fo);
  u32x4_t ring[kRing];
#pragma unroll
  for (int i = 0; i < kRing; ++i) ring[i] = ping_frag_at(fb, i);
  clear_s(st);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const bf16x8_t a = as_bf16x8(ring[i % kRing]);
    ping_mma<F16>(st, i, a);
    if (i + kRing < 32) ring[i % kRing] = ping_frag_at(fb, i + kRing);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// P(t) = 2^(S(t) c - m) as 16-bit MFMA fragments; sum[rb] = this lane's sum of row block rb's fp32 values.
template <bool F16>
BB_DEV void ping_exp(PingState& st, float c, float (&sum)[2]) {
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float nm = -st.m[rb];
#pragma unroll
    for (int stp = 0; stp < 2; ++stp) {
      float pe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pe[e] = fast_exp2(fmaf(st.s[2 * stp + e / 4][rb][e % 4], c, nm));
        sum[rb] = stp == 0 && e == 0 ? pe[e] : sum[rb] + pe[e];  // no 0 + p[0] add
      }
      st.pk[stp][rb] = as_bf16x8(u32x4_t{pack2<F16>(pe[0], pe[1]), pack2<F16>(pe[2], pe[3]),
                                         pack2<F16>(pe[4], pe[5]), pack2<F16>(pe[6], pe[7])});
    }
  }
}

// Tile maximum of S(t) over the 64 keys of row block rb's row, times c.
BB_DEV float ping_tile_max(const PingState& st, int rb, float c) {
  // NaN-propagating maximum (v_maximum3_f32): fmaxf would first canonicalise every MFMA result
  float mx = __builtin_elementwise_maximum(st.s[0][rb][0], st.s[1][rb][0]);
#pragma unroll
  for (int kb = 0; kb < 4; kb += 2)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (kb + i > 0) mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(st.s[kb][rb][i], st.s[kb + 1][rb][i]));
  return row4_max(mx) * c;
}

// Moves the exponent offset of row block rb to mt where `need`, rescaling its O and l.
BB_DEV void ping_rescale(PingState& st, int rb, bool need, float mt) {
  const float alpha = need ? fast_exp2(st.m[rb] - mt) : 1.0f;
  if (need) st.m[rb] = mt;
  st.l[rb] *= alpha;
#pragma unroll
  for (int db = 0; db < PD / 16; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) st.o[db][rb][i] *= alpha;
}

// Online softmax of a masked tile S(t) into P(t): running offset m (log2 units), sum l, O rescaled when the tile
// maximum exceeds m by more than kRescaleThreshold. bits(rb, kb) gives the 4 valid-key bits of key block kb for row
// block rb's row.
template <bool F16, typename Bits>
BB_DEV void ping_softmax_masked(PingState& st, float c, const Bits& bits) {
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint32_t b = bits(rb, kb);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!((b >> i) & 1u)) st.s[kb][rb][i] = -__builtin_huge_valf();
    }
  float mt[2];
  bool need[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    mt[rb] = ping_tile_max(st, rb, c);
    need[rb] = mt[rb] > st.m[rb] + kRescaleThreshold;  // the same on the row's four lanes
  }
  if (__builtin_amdgcn_ballot_w64(need[0] || need[1])) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) ping_rescale(st, rb, need[rb], mt[rb]);
  }
  float sum[2];
  ping_exp<F16>(st, c, sum);
  st.l[0] += sum[0];
  st.l[1] += sum[1];
}

// Online softmax of a tile with no masked element. The tile is exponentiated against the current offset first;
// only when a probability may exceed 2^kRescaleThreshold (a lane's partial sum of a row does: every term is at most
// that sum; an infinite or NaN sum counts too) is the tile maximum taken, the offset moved and the tile exponentiated
// again. Same bound on P as the masked form, without a maximum per tile in the common case.
template <bool F16>
BB_DEV void ping_softmax_open(PingState& st, float c) {
  float sum[2];
  ping_exp<F16>(st, c, sum);
  const float lim = __builtin_amdgcn_exp2f(kRescaleThreshold);
  const bool over0 = !(sum[0] <= lim), over1 = !(sum[1] <= lim);
  if (__builtin_amdgcn_ballot_w64(over0 || over1)) {  // some lane needs it: only then combine the row's lanes
    const bool need0 = row4_any(over0), need1 = row4_any(over1);
    const float mt0 = ping_tile_max(st, 0, c), mt1 = ping_tile_max(st, 1, c);
    // the new offset never goes below the old one, so rows that do not need it keep theirs
    ping_rescale(st, 0, need0, __builtin_elementwise_maximum(mt0, st.m[0]));
    ping_rescale(st, 1, need1, __builtin_elementwise_maximum(mt1, st.m[1]));
    ping_exp<F16>(st, c, sum);
  }
  st.l[0] += sum[0];
  st.l[1] += sum[1];
}

// Work item of a workgroup and the rows of one wave: (KV head, row tile of 32 x 8 / HPW rows, key chunk), XCD-aware as
// in flash_kernel.
struct PipeItem {
  int bh, kvbh, chunk;
  int64_t T_eff, r1, qlo, qhi, rw, qw0, qw1;
  bool wave_live;
};

template <int HPW>
BB_DEV PipeItem pipe_item(const FlashParams& p, int bid, int hd, int rbk) {
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
  const int x = lane & 15, a = lane >> 4;
  const int hd = wave % HPW, rbk = wave / HPW;  // head slot, row block
  const int grp = wave >> 2;                    // ping-pong group: waves w and w + 4 share a SIMD

  // ---- work item: (KV head, row tile), XCD-aware as in flash_kernel ----
  PipeItem it = pipe_item<HPW>(p, blockIdx.x, hd, rbk);
  const int bh = it.bh, kvbh = it.kvbh, chunk = it.chunk;
  const int64_t T_eff = it.T_eff, qlo = it.qlo, qhi = it.qhi, rw = it.rw;
  const bool wave_live = it.wave_live;
  const int64_t qw0 = it.qw0, qw1 = it.qw1;

  PingState st;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int64_t row = rw + 16 * rb + x;
    const bool live = row < T_eff;
    const uint16_t* qrow = p.q + (int64_t)bh * p.sq0 + (live ? row : T_eff - 1) * p.sq1 + 8 * a;
#pragma unroll
    for (int ds = 0; ds < PD / 32; ++ds) {
      const u32x4_t v = ld16(qrow + 32 * ds);
      st.qf[rb][ds] = as_bf16x8(live ? v : u32x4_t{0, 0, 0, 0});
    }
#pragma unroll
    for (int db = 0; db < PD / 16; ++db) st.o[db][rb] = zero4();
    st.m[rb] = -1.0e20f;
    st.l[rb] = 0.0f;
  }
  // this lane's query positions (row block rb: row 16 rb + x of the wave)
  const int64_t qx0 = qw0 + x * p.pos_step, qx1 = qx0 + 16 * p.pos_step;

  const uint16_t* kbase = p.k + (int64_t)kvbh * p.sk0;
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
  auto clip = [&](int64_t& lo, int64_t& hi) {
    if (lo < c0) lo = c0;
    if (hi > c1) hi = c1;
    if (hi < lo) hi = lo;
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
  // VALU phase of tile t: the masked softmax (front | causal window) for the edge tiles
  auto softmax_masked = [&](int t) {
    const int64_t k0 = upos(t), k1 = k0 + kTileKeys - 1;
    const bool live = wave_live && k0 <= qw1 && !(k0 >= p.front && k1 <= qw0 - p.window);
    const PipeWindowMask mk{k0, p.front, p.window, live};
    ping_softmax_masked<F16>(st, p.c, [&](int rb, int kb) { return mk.bits(rb ? qx1 : qx0, kb, a); });
  };
  auto softmax = [&](int t) {
    if (t < nu) ping_softmax_open<F16>(st, p.c);
    else softmax_masked(t);
  };

  uint16_t* ring = smem;
  auto kst = [&](int t) { return ring + (t & (PST - 1)) * 2 * PTE; };
  auto vst = [&](int t) { return ring + (t & (PST - 1)) * 2 * PTE + PTE; };
  const FragOfs fo = frag_ofs(x, a);
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
    ping_qk<F16>(st, kst(0), fo);
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
    ping_pv<F16>(st, vst(ntot - 1), fo);
    if (grp == 0) ring_barrier();  // realign the two groups
  }

  // The work item again, from copies of the block and lane indices that the compiler cannot see through: the values
  // the routed phase and the epilogue need are recomputed here instead of being held (and spilled) across the loop.
  {
    int bid2 = blockIdx.x;
    asm volatile("" : "+s"(bid2));
    it = pipe_item<HPW>(p, bid2, hd, rbk);
  }
  // ---- routed keys: per-head tiles pre-gathered by route_tiles_kernel; the RB waves of a head share the loads ----
  if (p.route_k > 0) {
    __syncthreads();  // every wave is done with the ring
    uint16_t* kl = smem + hd * 2 * PTE;
    uint16_t* vt = kl + PTE;
    int64_t g_first = it.qlo / p.route_chunk, g_last = it.qhi / p.route_chunk;
    if (g_last >= p.n_groups) g_last = p.n_groups - 1;
    const uint32_t loff = 16u * (uint32_t)lane;
    const int64_t qr0 = it.qw0 + x * p.pos_step, qr1 = qr0 + 16 * p.pos_step;
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
      // a routed key is usable by this lane's rows when key <= q - window and q lies in route group g
      auto route_lim = [&](int64_t q) -> int {
        const int64_t lim64 = q / p.route_chunk == g ? q - p.window : -1;
        return lim64 > 0x7fffffff ? 0x7fffffff : (lim64 < -1 ? -1 : (int)lim64);
      };
      const int lim0 = route_lim(qr0), lim1 = route_lim(qr1);
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
        for (int xh = 0; xh < HPW; ++xh)
#pragma unroll
          for (int y = 0; y < RB; ++y) {
            const int v = head_batches[y][xh];
            nb = nb > v ? nb : v;
            if (xh == hd) my_nb = my_nb > v ? my_nb : v;
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
            // units of 4 keys x 8 d into the V^T layout. Only batches holding a usable key are gathered.
            const uint16_t* kb = p.k + (int64_t)it.kvbh * p.sk0;
            const uint16_t* vb = p.v + (int64_t)it.kvbh * p.sv0;
            for (int b = rbk; b < PBLK; b += RB) {
              const int e = b * 512 + 8 * lane;
              const int row = e / PD, chk = ((e % PD) / 8) ^ pk_swz(row);
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
                *reinterpret_cast<u32x2_t*>(vt + pv_off(8 * bq + e, 2 * (a4 >> 2) + (a4 & 1)) + 4 * ((a4 >> 1) & 1)) =
                    u32x2_t{lo, hi};
              }
            }
          }
          vm_wait_tile(false);
          __syncthreads();
          if (work && it.wave_live) {
            // the list's keys of this lane's S^T elements: slots kblk_base(kb, a) + 0..3, one 16-byte read per block
            i32x4_t k4[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) k4[kb] = *reinterpret_cast<const i32x4_t*>(keys + kblk_base(kb, a));
            ping_qk<F16>(st, kl, fo);
            ping_softmax_masked<F16>(st, p.c, [&](int rb, int kb) {
              const int lim = rb ? lim1 : lim0;
              uint32_t bb = 0;
#pragma unroll
              for (int i = 0; i < 4; ++i) bb |= (uint32_t)(k4[kb][i] >= 0 && k4[kb][i] <= lim) << i;
              return bb;
            });
            ping_pv<F16>(st, vt, fo);
          }
          __syncthreads();
        }
      }
    }
  }

  // ---- epilogue ----
  if (p.route_k <= 0) __syncthreads();  // the ring is free for the output staging (the routed phase ends on one)
  if (!it.wave_live) return;
  const float lt[2] = {row4_sum(st.l[0]), row4_sum(st.l[1])};
  if (p.n_chunks > 1) {  // partial (O, m, l) of this key chunk for flash_merge_kernel
    // The fp32 rows pass through this wave's 16 KB of LDS (row r at r * 512 bytes, its 16-byte chunk k in slot
    // k ^ (r % 16)) so that every global store writes two whole rows, as for the output below.
    float* fstage = reinterpret_cast<float*>(smem) + wave * (32 * PD);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int r = 16 * rb + x;
#pragma unroll
      for (int db = 0; db < PD / 16; ++db) {
        const int k = 4 * db + a;  // d = 4k .. 4k + 3
        *reinterpret_cast<f32x4_t*>(fstage + r * PD + 4 * (k ^ (r & 15))) = st.o[db][rb];
      }
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
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int r = 16 * rb + x;
      if (a == 0 && it.rw + r < it.T_eff) {
        p.part_ml[2 * (base0 + r)] = st.m[rb];
        p.part_ml[2 * (base0 + r) + 1] = lt[rb];
      }
    }
    return;
  }
  // The normalised rows pass through this wave's 8 KB of LDS (row r at r * 256 bytes, its 16-byte chunk k in slot
  // k ^ (r % 16)), so that every global store writes two whole rows: lane l of store i takes bytes 8 (l % 32) .. of
  // row 2 i + l / 32. Stored from the fragment layout, each store would touch 16 rows.
  uint16_t* stage = smem + wave * (32 * PD);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float inv = 1.0f / fmaxf(lt[rb], 1.0e-20f);
    const int r = 16 * rb + x;
#pragma unroll
    for (int db = 0; db < PD / 16; ++db) {
      const int k = 2 * db + (a >> 1);  // 16-byte chunk of d = 16 db + 4 a .. + 3; half a & 1 of it
      const f32x4_t v = st.o[db][rb];
      const u32x2_t w = {pack2<F16>(v[0] * inv, v[1] * inv), pack2<F16>(v[2] * inv, v[3] * inv)};
      *reinterpret_cast<u32x2_t*>(stage + r * PD + 8 * (k ^ (r & 15)) + 4 * (a & 1)) = w;
    }
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
// LDS tile layouts of the main pass (K tile: pk_off; V^T tile: pv_off), so that the routed phase streams them with
// direct loads like window tiles. Empty slots (-1, or outside [0, N)) are zero rows. Grid (batches, n_groups, BH),
// 256 threads.
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
    st16(kt + pk_off(row, chunk), v);
  }
  // V^T tile: unit (4 keys x 8 d) per thread, transposed into the permuted key order of the V^T layout
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
    *reinterpret_cast<u32x2_t*>(vtt + pv_off(d, 2 * (a4 >> 2) + (a4 & 1)) + 4 * ((a4 >> 1) & 1)) = u32x2_t{lo, hi};
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
