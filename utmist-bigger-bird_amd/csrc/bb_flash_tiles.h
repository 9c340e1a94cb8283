// LDS tile layouts, direct global->LDS loads and mask helpers shared by the sparse flash kernels (gfx950).
#pragma once
#include "bb_common.h"
#include "bb_internal.h"

namespace bb {
namespace {

constexpr int kTileKeys = 64;
constexpr float kRescaleThreshold = 8.0f;  // log2 units

template <int D>
struct Layout {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per K row
  static constexpr int kKElems = kTileKeys * D;     // K tile: 64 rows x D, chunk slot = chunk ^ (row % CPR)
  static constexpr int kVElems = D * kTileKeys;     // V^T tile: D rows x 64 keys, slot = unit ^ vt_swz(d)
  static constexpr int kTileElems = kKElems + kVElems;
  static constexpr int kBlocks = kKElems * 2 / 1024;  // 1 KB direct-load blocks per K (or V^T) tile
};

template <int D>
BB_DEV int k_off(int row, int chunk) {
  return row * D + 8 * (chunk ^ (row & (Layout<D>::CPR - 1)));
}
// V^T layout. Inside every 16-key group a V^T row stores its keys in the order 0-3, 8-11, 4-7, 12-15 (bits 2 and 3
// of the key index swapped), so the 8 keys {4h..4h+3, 8+4h..8+4h+3} a lane feeds to the PV MFMA form one 16-byte unit
// (unit 2g + h of a 64-key tile row, g the 16-key group). In LDS, unit u of row d sits in 16-byte slot u ^ vt_swz(d):
// the fragment reads of 32 consecutive rows by a wave then touch every bank once per LDS cycle.
BB_DEV int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }
BB_DEV int vt_off(int d, int unit) { return d * kTileKeys + 8 * (unit ^ vt_swz(d)); }
// element offset, inside a tile row, of key kk's value (the 16-key group permutation above)
__host__ __device__ inline int vt_key_pos(int kk) { return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1); }

BB_DEV void lds_dma16(const void* g, uint16_t* lds) {
  __builtin_amdgcn_global_load_lds(g, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                          reinterpret_cast<uintptr_t>(lds)),
                                   16, 0, 0);
}

BB_DEV void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Issue direct loads of one window tile (K rows k0..k0+63, V^T columns k0..k0+63). Block b of the K (V^T) tile is
// written by wave b % NW; lane l of a block lands at byte 16 * l of it.
template <int D, int NW>
BB_DEV void issue_window_tile(uint16_t* kl, uint16_t* vt, const uint16_t* kbase, int64_t sk1, const uint16_t* vtbase,
                              int64_t np, int64_t k0, int64_t N, int wave, int lane) {
  for (int b = wave; b < Layout<D>::kBlocks; b += NW) {
    const int e = b * 512 + 8 * lane;
    const int row = e / D, slot = (e % D) / 8;
    const int chunk = slot ^ (row & (Layout<D>::CPR - 1));
    int64_t pos = k0 + row;
    if (pos >= N) pos = N - 1;  // clamped rows are masked out
    lds_dma16(kbase + pos * sk1 + 8 * chunk, kl + b * 512);
  }
  for (int b = wave; b < Layout<D>::kBlocks; b += NW) {
    const int d = 8 * b + lane / 8, slot = lane % 8;
    const int chunk = slot ^ vt_swz(d);
    lds_dma16(vtbase + (int64_t)d * np + k0 + 8 * chunk, vt + b * 512);
  }
}

template <int D, int QB>
struct WaveState {
  bf16x8_t qf[QB][D / 16];
  f32x16_t o[QB][D / 32];
  float m[QB];
  float l[QB];
};

BB_DEV int clamp64(int64_t x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : (int)x); }

// Window/front mask of one tile for one query row, reduced to int32 thresholds on the tile-relative key kk:
// valid iff kk <= causal && kk < in_n && (kk < front || kk > win).
struct WindowMask {
  int64_t k0, N, front, window;
  const uint8_t* km;
  struct Row {
    int causal, in_n, front, win;
    const uint8_t* km;
    BB_DEV bool operator()(int kk) const {
      bool ok = kk <= causal && kk < in_n && (kk < front || kk > win);
      if (km) ok = ok && km[kk];
      return ok;
    }
  };
  BB_DEV Row row(int64_t q) const {
    return Row{clamp64(q - k0, -1, kTileKeys), clamp64(N - k0, 0, kTileKeys), clamp64(front - k0, 0, kTileKeys),
               clamp64(q - window - k0, -1, kTileKeys), km ? km + k0 : nullptr};
  }
};

// Routed mask: gathered key kk (LDS list, -1 = empty) is valid iff key <= q - window and q is in this route group.
struct RoutedMask {
  const int32_t* keys;
  int64_t window, route_chunk, group;
  const uint8_t* km;
  struct Row {
    const int32_t* keys;
    int lim;
    bool grp;
    const uint8_t* km;
    BB_DEV bool operator()(int kk) const {
      const int key = keys[kk];
      bool ok = grp && key >= 0 && key <= lim;
      if (km) ok = ok && km[key >= 0 ? key : 0];
      return ok;
    }
  };
  BB_DEV Row row(int64_t q) const {
    const int64_t lim = q - window;
    return Row{keys, lim > 0x7fffffff ? 0x7fffffff : (lim < -1 ? -1 : (int)lim), q / route_chunk == group, km};
  }
};

}  // namespace
}  // namespace bb
