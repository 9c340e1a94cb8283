// C ABI of libbb_attn: argument validation (reference error texts), schedule selection, kernel launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "bb_attn.h"
#include "bb_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return BB_EINVAL;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return BB_OK;
  snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return BB_EHIP;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Work schedule of the sparse flash kernel.
struct FlashSchedule {
  int hpw, head_splits, row_tiles, n_chunks;
  int64_t key_chunk;
  bool split;
};

constexpr int kCUs = 256;

// The software-pipelined main-pass kernel is used wherever it applies; BB_FLASH_PIPE=0 selects the generic kernel
// (for measurement).
bool flash_pipe_enabled() {
  static bool on = [] {
    const char* e = getenv("BB_FLASH_PIPE");
    return !(e && e[0] == '0');
  }();
  return on;
}

FlashSchedule flash_schedule(int BH, int64_t T, int64_t N, int num_heads, int kv_groups, int64_t front, int64_t window,
                             int route_k, int64_t row_end) {
  FlashSchedule s;
  const int G = kv_groups;
  s.hpw = (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
  s.head_splits = G / s.hpw;
  const int64_t R = 64 * (4 / s.hpw);
  const int64_t rows = row_end < T ? row_end : T;
  s.row_tiles = (int)cdiv(rows > 0 ? rows : 0, R);
  const int64_t n_kvbh = BH / G;
  const int64_t items = n_kvbh * s.head_splits * s.row_tiles;
  int64_t span = (window < N ? window : N) + R;  // keys per item (window part)
  s.split = false;
  s.n_chunks = 1;
  s.key_chunk = N;
  (void)front;
  (void)num_heads;
  // Few long items (the exact tail: a few row tiles over every key) are cut into key chunks until the grid fills the
  // chip once: one workgroup fits a CU, and a second round of workgroups costs a second prologue and epilogue (the
  // 128K tail 0.47 -> 0.44 ms with 8 chunks instead of 16).
  if (route_k == 0 && items > 0 && items < 2 * kCUs && span / 64 > 32) {
    int64_t want = cdiv(kCUs, items);
    int64_t max_chunks = cdiv(N, 4096);
    int64_t nc = want < max_chunks ? want : max_chunks;
    if (nc > 1) {
      s.key_chunk = cdiv(cdiv(N, nc), 64) * 64;
      s.n_chunks = (int)cdiv(N, s.key_chunk);
      s.split = s.n_chunks > 1;
      if (!s.split) {
        s.n_chunks = 1;
        s.key_chunk = N;
      }
    }
  }
  return s;
}

// Static scratch of bb_decode_noalloc: the split partials [H][n_splits][D + 2] fp32 live in this array instead of a
// caller workspace. Every GPU the library runs on holds its own copy for the life of the process; calls that overlap
// on one GPU share it and race. Host code never passes `decode_scratch_mem` itself (that name is a host-side
// stand-in): its device address comes from hipGetSymbolAddress, looked up once per device with that device current.
constexpr size_t kDecodeScratchBytes = (size_t)2 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char decode_scratch_mem[kDecodeScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of the current device's scratch (looked up on the first call on that device).
int decode_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "bb_decode_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail("decode_noalloc: device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* addr = nullptr;
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(decode_scratch_mem));
    if (e != hipSuccess) return hip_status(e, "bb_decode_noalloc: hipGetSymbolAddress");
    if (!addr) return fail("decode_noalloc: no device address for the scratch array");
    g_scratch_addr[dev] = addr;
  }
  *out = g_scratch_addr[dev];
  return BB_OK;
}

}  // namespace

extern "C" {

int bb_version(void) { return BB_ABI_VERSION; }

// Per-device set-up done ahead of time: the device address of bb_decode_noalloc's static scratch, so that the entry
// point's first call on this device (which may sit inside a HIP graph capture) does no symbol lookup.
int bb_init(void) {
  g_err[0] = 0;
  void* addr = nullptr;
  return decode_scratch(&addr);
}

const char* bb_last_error(void) { return g_err; }

int64_t bb_transpose_v_cols(int64_t N) { return cdiv(N > 0 ? N : 1, 64) * 64; }

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Routed tiles are pre-gathered for the pipelined kernel (head_dim 128, query heads per KV head a multiple of 4, no
// token mask) when the route list has a single group. With several groups (vertical_scope) most groups are empty and
// the tiles of every group would cost BH x groups x 32 KB per 64 slots, so the kernel gathers the batches it uses
// itself. K rows of 4 GiB or more per KV head also leave the pipelined kernel; the reservation does not see the row
// stride and is made anyway (it is small next to such K).
static bool routed_tiles_wanted(int D, int kv_groups, int route_k, int n_groups, bool key_mask) {
  return route_k > 0 && n_groups == 1 && !key_mask && D == 128 && kv_groups > 0 && flash_pipe_enabled();
}

size_t bb_sparse_flash_workspace(int BH, int64_t T, int64_t N, int D, int num_heads, int kv_groups, int64_t front,
                                 int64_t window, int route_k, int n_groups, int64_t row_end, int have_vt,
                                 int has_key_mask) {
  if (BH <= 0 || T <= 0 || N <= 0 || kv_groups <= 0 || BH % kv_groups) return 0;
  if (window >= N) route_k = 0;
  if (row_end <= 0 || row_end > T) row_end = T;
  FlashSchedule s = flash_schedule(BH, T, N, num_heads, kv_groups, front, window, route_k, row_end);
  size_t bytes = 0;
  if (!have_vt) bytes += align256((size_t)(BH / kv_groups) * D * bb_transpose_v_cols(N) * 2);
  if (routed_tiles_wanted(D, kv_groups, route_k, n_groups, has_key_mask != 0))
    bytes += align256(bb::route_tiles_bytes(BH, n_groups, route_k));
  if (s.split) bytes += (size_t)s.n_chunks * BH * T * (size_t)(D + 2) * sizeof(float);
  return bytes;
}

int bb_transpose_v(const void* v, const int64_t* sv, int n_kvbh, int64_t N, int D, void* vt, void* stream) {
  g_err[0] = 0;
  if (!v || !sv || !vt) return fail("transpose_v: null argument");
  if (D != 32 && D != 64 && D != 128) return fail("head_dim %d unsupported (32, 64 or 128)", D);
  if (!aligned(v, 16) || !aligned(vt, 16) || sv[0] % 8 || sv[1] % 8 || sv[2] != 1)
    return fail("q/k/v need a contiguous head_dim and 16-byte aligned rows");
  return hip_status(bb::launch_transpose_v(static_cast<const uint16_t*>(v), sv[0], sv[1], n_kvbh, N,
                                           bb_transpose_v_cols(N), D, static_cast<uint16_t*>(vt),
                                           static_cast<hipStream_t>(stream)),
                    "bb_transpose_v");
}

// bb_sparse_flash, and with `noncausal` the exact attention of every query row over all N keys (bb_exact_attention:
// front 0, window N, no routes, every row placed at position N - 1).
static int sparse_flash_impl(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                             const int64_t* sv, const void* vt, const int32_t* idx, const int64_t* si, int n_groups,
                             int route_k, const uint8_t* key_mask, int64_t smb, void* out, const int64_t* so, int BH,
                             int64_t T, int64_t N, int D, int is_f16, int num_heads, int kv_groups, int64_t front,
                             int64_t window, int64_t route_chunk, float scale, int64_t row_end, void* ws,
                             size_t ws_bytes, void* stream, bool noncausal) {
  g_err[0] = 0;
  if (!q || !k || !v || !out || !sq || !sk || !sv || !so)
    return fail("Q [BH,T,D] and K/V [BH/kv_groups,N,D] must have matching heads and dimensions");
  if (kv_groups <= 0 || num_heads <= 0 || BH <= 0 || BH % kv_groups || num_heads % kv_groups || BH % num_heads)
    return fail("Q [BH,T,D] and K/V [BH/kv_groups,N,D] must have matching heads and dimensions");
  if (D != 32 && D != 64 && D != 128) return fail("head_dim %d unsupported (32, 64 or 128)", D);
  if (front < 0 || window < 1) return fail("front >= 0 and window >= 1 required");
  if (T > N) return fail("Key sequence must be at least as long as query sequence");
  if (T <= 0) return BB_OK;
  if (route_k < 0 || (route_k > 0 && (!idx || !si || n_groups <= 0)))
    return fail("Routing groups must cover the sequence and align with query tiles");
  if (route_chunk <= 0 || (route_k > 0 && n_groups != cdiv(N, route_chunk)))
    return fail("Routing groups must cover the sequence and align with query tiles");
  if (!(scale > 0.0f)) return fail("scale must be positive");
  // 16-byte operand loads, 8-byte output stores
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || sq[0] % 8 || sq[1] % 8 || sk[0] % 8 || sk[1] % 8 ||
      sv[0] % 8 || sv[1] % 8 || sq[2] != 1 || sk[2] != 1 || sv[2] != 1)
    return fail("q/k/v need a contiguous head_dim and 16-byte aligned rows");
  if (!aligned(out, 8) || so[0] % 4 || so[1] % 4 || so[2] != 1)
    return fail("out needs a contiguous head_dim and 8-byte aligned rows");
  if (front > N) front = N;
  if (row_end <= 0 || row_end > T) row_end = T;

  // A routed key j is attended only when j <= q - window; with window >= N no key qualifies, so the routes are
  // dropped (this is how the exact tail calls the kernel: window = N with a -1 route list).
  if (window >= N) route_k = 0;
  FlashSchedule s = flash_schedule(BH, T, N, num_heads, kv_groups, front, window, route_k, row_end);
  bb::FlashParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.idx = idx;
  p.key_mask = key_mask;
  p.out = static_cast<uint16_t*>(out);
  p.sq0 = sq[0]; p.sq1 = sq[1];
  p.sk0 = sk[0]; p.sk1 = sk[1];
  p.sv0 = sv[0]; p.sv1 = sv[1];
  if (si) { p.si0 = si[0]; p.si1 = si[1]; p.si2 = si[2]; }
  p.smb = smb;
  p.so0 = so[0]; p.so1 = so[1];
  p.N = N; p.T = T; p.row_end = row_end;
  p.f16 = is_f16 ? 1 : 0;
  p.offset = noncausal ? N - 1 : N - T;
  p.pos_step = noncausal ? 0 : 1;
  p.route_chunk = route_chunk;
  p.key_chunk = s.key_chunk;
  p.BH = BH; p.H = num_heads; p.G = kv_groups; p.Hkv_pb = num_heads / kv_groups; p.n_kvbh = BH / kv_groups;
  p.front = (int)front;
  p.window = (int)(window > N + 1 ? N + 1 : window);
  p.route_k = route_k;
  p.n_groups = n_groups > 0 ? n_groups : 1;
  p.row_tiles = s.row_tiles;
  p.head_splits = s.head_splits;
  p.n_chunks = s.n_chunks;
  p.remap = ((int64_t)p.n_kvbh * s.head_splits) % 8 == 0;
  p.np = bb_transpose_v_cols(N);
  p.c = (float)((double)scale * 1.4426950408889634);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t need = bb_sparse_flash_workspace(BH, T, N, D, num_heads, kv_groups, front, window, route_k, p.n_groups,
                                                row_end, vt != nullptr, key_mask != nullptr);
  if (need && (!ws || ws_bytes < need)) return fail("workspace of %zu bytes required", need);
  char* wsp = static_cast<char*>(ws);
  if (vt) {
    if (!aligned(vt, 16)) return fail("vt must be 16-byte aligned");
    p.vt = static_cast<const uint16_t*>(vt);
  } else {
    uint16_t* vt_ws = reinterpret_cast<uint16_t*>(wsp);
    wsp += align256((size_t)p.n_kvbh * D * p.np * 2);
    hipError_t e = bb::launch_transpose_v(p.v, p.sv0, p.sv1, p.n_kvbh, N, p.np, D, vt_ws, st);
    if (e != hipSuccess) return hip_status(e, "bb_sparse_flash transpose");
    p.vt = vt_ws;
  }
  const bool pipe = flash_pipe_enabled() && bb::flash_pipe_supported(p, D, s.hpw);
  if (routed_tiles_wanted(D, kv_groups, route_k, p.n_groups, key_mask != nullptr)) {
    uint16_t* rt = reinterpret_cast<uint16_t*>(wsp);
    wsp += align256(bb::route_tiles_bytes(BH, p.n_groups, route_k));
    if (pipe) {
      p.rtiles = rt;
      p.rt_batches = (int)cdiv(route_k, 64);
      hipError_t e = bb::launch_route_tiles(p, rt, st);
      if (e != hipSuccess) return hip_status(e, "bb_sparse_flash routed tiles");
    }
  }
  if (s.split) {
    p.part_o = reinterpret_cast<float*>(wsp);
    p.part_ml = p.part_o + (size_t)s.n_chunks * BH * T * D;
    hipError_t e = pipe ? bb::launch_flash_pipe(p, s.hpw, st) : bb::launch_flash(p, D, s.hpw, true, st);
    if (e != hipSuccess) return hip_status(e, "bb_sparse_flash split kernel");
    return hip_status(bb::launch_flash_merge(p, D, st), "bb_sparse_flash merge kernel");
  }
  if (pipe) return hip_status(bb::launch_flash_pipe(p, s.hpw, st), "bb_sparse_flash pipelined kernel");
  return hip_status(bb::launch_flash(p, D, s.hpw, false, st), "bb_sparse_flash kernel");
}

int bb_sparse_flash(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                    const int64_t* sv, const void* vt, const int32_t* idx, const int64_t* si, int n_groups,
                    int route_k, const uint8_t* key_mask, int64_t smb, void* out, const int64_t* so, int BH, int64_t T,
                    int64_t N, int D, int is_f16, int num_heads, int kv_groups, int64_t front, int64_t window,
                    int64_t route_chunk, float scale, int64_t row_end, void* ws, size_t ws_bytes, void* stream) {
  return sparse_flash_impl(q, sq, k, sk, v, sv, vt, idx, si, n_groups, route_k, key_mask, smb, out, so, BH, T, N, D,
                           is_f16, num_heads, kv_groups, front, window, route_chunk, scale, row_end, ws, ws_bytes,
                           stream, false);
}

size_t bb_exact_attention_workspace(int BH, int64_t T, int64_t N, int D, int num_heads, int kv_groups, int have_vt) {
  return bb_sparse_flash_workspace(BH, T, N, D, num_heads, kv_groups, 0, N, 0, 1, T, have_vt, 0);
}

int bb_exact_attention(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                       const int64_t* sv, const void* vt, void* out, const int64_t* so, int BH, int64_t T, int64_t N,
                       int D, int is_f16, int num_heads, int kv_groups, float scale, void* ws, size_t ws_bytes,
                       void* stream) {
  const int64_t si[3] = {0, 0, 0};
  return sparse_flash_impl(q, sq, k, sk, v, sv, vt, nullptr, si, 1, 0, nullptr, 0, out, so, BH, T, N, D, is_f16,
                           num_heads, kv_groups, 0, N, N, scale, T, ws, ws_bytes, stream, true);
}

size_t bb_routes_workspace(int64_t n, int H, int Hkv, int B, int r) {
  if (n <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || B <= 0 || r <= 0) return 0;
  return bb::routes_workspace_bytes(n, H, Hkv, B, r);
}

// BB_ROUTES_REFERENCE_ORDER=1 computes every route score with the reference-order chain instead of MFMA + exact
// fix-up (same results by construction; the switch exists to cross-check that).
static int routes_reference_order() {
  const char* e = getenv("BB_ROUTES_REFERENCE_ORDER");
  return e && e[0] == '1';
}

int bb_routes(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const int64_t* qpos, int r, int B,
              int H, int Hkv, int64_t n, int D, int is_f16, int64_t sink, int64_t window, int budget, float scaling,
              int pool_max, int32_t* idx_out, uint64_t* pooled_out, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (!q || !k || !qpos || !sq || !sk) return fail("routes: null argument");
  if (H <= 0 || Hkv <= 0 || H % Hkv || B <= 0 || n <= 0 || r <= 0) return fail("routes: bad head/sequence sizes");
  if (D != 32 && D != 64 && D != 128) return fail("head_dim %d unsupported (32, 64 or 128)", D);
  if (H / Hkv * r > 4096) return fail("routes: groups * n_route must be <= 4096");
  if (!aligned(q, 16) || !aligned(k, 16) || sq[0] % 8 || sq[1] % 8 || sk[0] % 8 || sk[1] % 8)
    return fail("q/k need a contiguous head_dim and 16-byte aligned rows");
  int64_t lo = sink < n ? (sink > 0 ? sink : 0) : n;
  int64_t hi = n - window;
  if (hi > n) hi = n;
  const int64_t eligible = hi > lo ? hi - lo : 0;
  if (budget < 0 || budget > eligible) return fail("routes: budget %d exceeds %lld eligible columns", budget, (long long)eligible);
  if (budget > 0 && !idx_out) return fail("routes: idx_out required");
  if (!(scaling > 0.0f)) return fail("scaling must be positive");
  const size_t need = bb::routes_workspace_bytes(n, H, Hkv, B, r);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  bb::RoutesParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.qpos = qpos;
  p.sq0 = sq[0]; p.sq1 = sq[1]; p.sk0 = sk[0]; p.sk1 = sk[1];
  p.n = n; p.H = H; p.Hkv = Hkv; p.B = B; p.D = D; p.r = r;
  p.sink = (int)(sink < n ? sink : n);
  p.window = (int)(window < n ? window : n);
  p.budget = budget; p.pool_max = pool_max; p.scaling = scaling;
  p.out_idx = idx_out;
  p.scores_reference_order = routes_reference_order();
  p.f16 = is_f16 ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = bb::launch_routes(p, ws, ws_bytes, st);
  if (e != hipSuccess) return hip_status(e, "bb_routes");
  if (pooled_out) {
    e = hipMemcpyAsync(pooled_out, p.pooled, (size_t)B * H * n * sizeof(uint64_t), hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return hip_status(e, "bb_routes pooled copy");
  }
  return BB_OK;
}

int bb_int8_quantize(const void* x, int x_kind, int64_t outer, int64_t row_stride, int inner, int64_t inner_stride,
                     int D, float min_scale, int8_t* q, void* scale, int scale_is_f16, void* stream) {
  g_err[0] = 0;
  if (!x || !q || !scale) return fail("quantize: null argument");
  if (D != 32 && D != 64 && D != 128 && D != 256) return fail("quantize: head_dim %d unsupported", D);
  if (x_kind < 0 || x_kind > 2) return fail("quantize: element kind %d unsupported (0 bf16, 1 fp32, 2 fp16)", x_kind);
  const int64_t el = x_kind == 1 ? 4 : 2;
  if (!aligned(x, 16) || (row_stride * el) % 16 || (inner_stride * el) % 16 || !aligned(q, 8))
    return fail("quantize: rows must be 16-byte aligned");
  return hip_status(bb::launch_int8_quantize(x, x_kind, outer, row_stride, inner, inner_stride, D, min_scale, q, scale,
                                             scale_is_f16, static_cast<hipStream_t>(stream)),
                    "bb_int8_quantize");
}

int bb_int8_quantize_pair(const void* xk, const void* xv, int x_kind, int64_t outer, int64_t row_stride, int inner,
                          int64_t inner_stride, int D, float min_scale, int8_t* qk, void* sk, int8_t* qv, void* sv,
                          int scale_is_f16, void* stream) {
  g_err[0] = 0;
  if (!xk || !xv || !qk || !sk || !qv || !sv) return fail("quantize: null argument");
  if (D != 32 && D != 64 && D != 128 && D != 256) return fail("quantize: head_dim %d unsupported", D);
  if (x_kind < 0 || x_kind > 2) return fail("quantize: element kind %d unsupported (0 bf16, 1 fp32, 2 fp16)", x_kind);
  const int64_t el = x_kind == 1 ? 4 : 2;
  if (!aligned(xk, 16) || !aligned(xv, 16) || (row_stride * el) % 16 || (inner_stride * el) % 16 || !aligned(qk, 8) ||
      !aligned(qv, 8))
    return fail("quantize: rows must be 16-byte aligned");
  return hip_status(bb::launch_int8_quantize(xk, x_kind, outer, row_stride, inner, inner_stride, D, min_scale, qk, sk,
                                             scale_is_f16, static_cast<hipStream_t>(stream), xv, qv, sv),
                    "bb_int8_quantize_pair");
}

int bb_int8_dequantize(const int8_t* q, const void* scale, int scale_is_f16, int64_t rows, int D, void* out,
                       int out_kind, void* stream) {
  g_err[0] = 0;
  if (!q || !scale || !out) return fail("dequantize: null argument");
  if (D != 32 && D != 64 && D != 128 && D != 256) return fail("dequantize: head_dim %d unsupported", D);
  if (out_kind < 0 || out_kind > 2) return fail("dequantize: element kind %d unsupported (0 bf16, 1 fp32, 2 fp16)", out_kind);
  if (!aligned(q, 8) || !aligned(out, 16)) return fail("dequantize: misaligned buffers");
  return hip_status(bb::launch_int8_dequantize(q, scale, scale_is_f16, rows, D, out, out_kind,
                                               static_cast<hipStream_t>(stream)),
                    "bb_int8_dequantize");
}

// Keys per decode workgroup: two workgroups per CU of equal length (at least 256 keys), i.e. every workgroup resident
// at once (two fit a CU by LDS); four per CU ran as two rounds and measured 1.2 us slower per configs[4] step. The
// length is not rounded: the bytes per CU, not the 32-key chunks per wave, set the time of this HBM-bound kernel
// (rounding 131073 keys up to 1152 per split left 912 workgroups, some CUs with a third more bytes than others).
static int64_t decode_split_len(int64_t n, int Hkv) {
  int64_t len = cdiv(n, cdiv(2 * kCUs, Hkv));
  return len < 256 ? 256 : len;
}
static int decode_splits(int64_t n, int Hkv) { return (int)cdiv(n, decode_split_len(n, Hkv)); }

size_t bb_decode_workspace(int64_t n, int H, int Hkv, int D) {
  if (n <= 0 || Hkv <= 0) return 0;
  return bb::decode_workspace_bytes(H, D, decode_splits(n, Hkv));
}

// Argument checks and launch descriptor shared by bb_decode and bb_decode_noalloc (p.part is left to the caller).
static int decode_params(const void* q, int64_t sq, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
                         int scale_is_f16, const void* kb, const int64_t* skb, const void* vb, const int64_t* svb,
                         int64_t n, int H, int Hkv, int D, float scale, void* out, int64_t so, bb::DecodeParams& p) {
  if (!q || !out) return fail("decode: null argument");
  if (n <= 0) return fail("decode: empty cache");
  if (H <= 0 || Hkv <= 0 || H % Hkv) return fail("q [H,D] and k/v [Hkv,N,D] must match");
  const int G = H / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail("decode: groups %d unsupported", G);
  if (D != 64 && D != 128) return fail("decode: head_dim %d unsupported (64 or 128)", D);
  const bool int8 = k8 != nullptr;
  if (int8 && (!v8 || !ks || !vs)) return fail("decode: int8 cache needs k8, v8 and scales");
  if (!int8 && (!kb || !vb || !skb || !svb)) return fail("decode: bf16 cache needs kb, vb and strides");
  if (int8 && (!aligned(k8, 16) || !aligned(v8, 16))) return fail("decode: misaligned cache");
  if (!int8 && (!aligned(kb, 16) || !aligned(vb, 16) || skb[0] % 8 || skb[1] % 8 || svb[0] % 8 || svb[1] % 8))
    return fail("decode: misaligned cache");
  if (!(scale > 0.0f)) return fail("scale must be positive");
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.sq = sq;
  p.k8 = k8; p.v8 = v8; p.ks = ks; p.vs = vs;
  p.kb = static_cast<const uint16_t*>(kb);
  p.vb = static_cast<const uint16_t*>(vb);
  if (skb) { p.skb0 = skb[0]; p.skb1 = skb[1]; }
  if (svb) { p.svb0 = svb[0]; p.svb1 = svb[1]; }
  p.n = n; p.H = H; p.Hkv = Hkv; p.D = D; p.scale_is_f16 = scale_is_f16;
  p.split_len = decode_split_len(n, Hkv);
  p.n_splits = decode_splits(n, Hkv);
  p.c = (float)((double)scale * 1.4426950408889634);
  p.out = static_cast<uint16_t*>(out);
  p.so = so;
  return BB_OK;
}

int bb_decode(const void* q, int64_t sq, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
              int scale_is_f16, const void* kb, const int64_t* skb, const void* vb, const int64_t* svb, int64_t n,
              int H, int Hkv, int D, float scale, void* out, int64_t so, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  bb::DecodeParams p;
  const int rc = decode_params(q, sq, k8, ks, v8, vs, scale_is_f16, kb, skb, vb, svb, n, H, Hkv, D, scale, out, so, p);
  if (rc != BB_OK) return rc;
  const size_t need = bb::decode_workspace_bytes(H, D, p.n_splits);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  p.part = static_cast<float*>(ws);
  return hip_status(bb::launch_decode(p, static_cast<hipStream_t>(stream)), "bb_decode");
}

int bb_decode_append(const void* q, int64_t sq, int8_t* k8, void* ks, int8_t* v8, void* vs, int scale_is_f16,
                     const void* knew, int64_t sknew, const void* vnew, int64_t svnew, float min_scale, int64_t n,
                     int H, int Hkv, int D, float scale, void* out, int64_t so, void* ws, size_t ws_bytes,
                     void* stream) {
  g_err[0] = 0;
  if (!knew || !vnew || !k8 || !v8 || !ks || !vs) return fail("decode_append: null argument");
  if (!aligned(knew, 16) || !aligned(vnew, 16) || sknew % 8 || svnew % 8)
    return fail("decode_append: new rows need a contiguous head_dim and 16-byte aligned heads");
  if (!(min_scale > 0.0f)) return fail("decode_append: min_scale must be positive");
  bb::DecodeParams p;
  const int rc = decode_params(q, sq, k8, ks, v8, vs, scale_is_f16, nullptr, nullptr, nullptr, nullptr, n, H, Hkv, D,
                               scale, out, so, p);
  if (rc != BB_OK) return rc;
  const size_t need = bb::decode_workspace_bytes(H, D, p.n_splits);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  p.part = static_cast<float*>(ws);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t r0 = (n - 1) * Hkv;  // first (row, head) of the new token
  const size_t sbytes = scale_is_f16 ? 2 : 4;
  if (bb::decode_fuses_append(p)) {
    p.knew = static_cast<const uint16_t*>(knew);
    p.vnew = static_cast<const uint16_t*>(vnew);
    p.sknew = sknew; p.svnew = svnew;
    p.min_scale = min_scale;
    p.wk8 = k8; p.wv8 = v8; p.wks = ks; p.wvs = vs;
    return hip_status(bb::launch_decode(p, st), "bb_decode_append");
  }
  // other shapes: quantise the two rows in one launch when their strides agree, then decode
  hipError_t e;
  if (sknew == svnew)
    e = bb::launch_int8_quantize(knew, 0, 1, 0, Hkv, sknew, D, min_scale, k8 + r0 * D,
                                 static_cast<char*>(ks) + r0 * sbytes, scale_is_f16, st, vnew, v8 + r0 * D,
                                 static_cast<char*>(vs) + r0 * sbytes);
  else {
    e = bb::launch_int8_quantize(knew, 0, 1, 0, Hkv, sknew, D, min_scale, k8 + r0 * D,
                                 static_cast<char*>(ks) + r0 * sbytes, scale_is_f16, st);
    if (e == hipSuccess)
      e = bb::launch_int8_quantize(vnew, 0, 1, 0, Hkv, svnew, D, min_scale, v8 + r0 * D,
                                   static_cast<char*>(vs) + r0 * sbytes, scale_is_f16, st);
  }
  if (e != hipSuccess) return hip_status(e, "bb_decode_append quantize");
  return hip_status(bb::launch_decode(p, st), "bb_decode_append");
}

size_t bb_decode_noalloc_max_bytes(void) { return kDecodeScratchBytes; }

int bb_decode_noalloc(const void* q, int64_t sq, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
                      int scale_is_f16, const void* kb, const int64_t* skb, const void* vb, const int64_t* svb,
                      int64_t n, int H, int Hkv, int D, float scale, void* out, int64_t so, void* stream) {
  g_err[0] = 0;
  bb::DecodeParams p;
  const int rc = decode_params(q, sq, k8, ks, v8, vs, scale_is_f16, kb, skb, vb, svb, n, H, Hkv, D, scale, out, so, p);
  if (rc != BB_OK) return rc;
  const size_t need = bb::decode_workspace_bytes(H, D, p.n_splits);
  if (need > kDecodeScratchBytes)
    return fail("decode_noalloc: %zu bytes of split partials exceed the static scratch of %zu bytes (use bb_decode "
                "with a workspace)", need, (size_t)kDecodeScratchBytes);
  void* scratch_ptr = nullptr;
  const int src = decode_scratch(&scratch_ptr);
  if (src != BB_OK) return src;
  p.part = static_cast<float*>(scratch_ptr);
  return hip_status(bb::launch_decode(p, static_cast<hipStream_t>(stream)), "bb_decode_noalloc");
}

// Key chunks of the split-K decode kernels, as kernels/bigger_bird_decode.py:84-88 and bigger_bird_route.py:91-94
// choose them (64-key blocks, about four workgroups per CU; `splits` > 0 requests a count).
// Keys per split of a decode-time key range: `splits` when given, else about `per_cu` workgroups per CU over all
// `programs` rows (at least 256 keys each), not rounded, so that every workgroup reads the same number of keys. The
// split-K decode runs best at 2 per CU (fewer, longer splits: less per-workgroup set-up and a cheaper merge; 5.3 TB/s
// over a 128K-token bf16 cache), the routing scores pass at 4.
static int64_t decode_chunk_len(int64_t total, int programs, int splits, int64_t cap_splits, int per_cu = 2) {
  if (total <= 0) return 64;
  int64_t s = splits > 0 ? splits
                         : std::max<int64_t>(1, std::min<int64_t>(cdiv(total, 4 * 64), cdiv(per_cu * kCUs, programs)));
  if (cap_splits > 0 && s > cap_splits) s = cap_splits;
  return cdiv(total, s);
}

size_t bb_sparse_decode_workspace(int H, int Hkv, int D, int rows, int front, int window, int route_k, int splits) {
  if (H <= 0 || Hkv <= 0 || rows <= 0 || D <= 0) return 0;
  const int64_t total = (int64_t)front + window + route_k;
  const int64_t len = decode_chunk_len(total, rows, splits, 0);
  return (size_t)H * (size_t)cdiv(total > 0 ? total : 1, len) * (size_t)(D + 2) * sizeof(float);
}

int bb_sparse_decode(const void* q, int64_t sq, const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                     const int32_t* idx, const int64_t* si, int rows, int route_k, int64_t n, const int64_t* n_dev,
                     int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                     void* out, int64_t so, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (!q || !k || !v || !sk || !sv || !out) return fail("q [H,D] and k/v [Hkv,N,D] must match");
  if (H <= 0 || Hkv <= 0 || H % Hkv || cap <= 0) return fail("q [H,D] and k/v [Hkv,N,D] must match");
  const int G = H / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail("decode: groups %d unsupported", G);
  if (D != 64 && D != 128) return fail("decode: head_dim %d unsupported (64 or 128)", D);
  if (rows != Hkv && rows != H) return fail("indices must be [Hkv, R] (pooled) or [H, R] (per head)");
  if (route_k < 0 || (route_k > 0 && (!idx || !si))) return fail("indices must be [Hkv, R] (pooled) or [H, R] (per head)");
  if (front < 0 || window < 0) return fail("front >= 0 and window >= 0 required");
  if (!n_dev && cap < (int64_t)front + window) return fail("cache shorter than front + window: use dense attention");
  if (!(scale > 0.0f)) return fail("scale must be positive");
  if (!aligned(q, 2) || !aligned(k, 16) || !aligned(v, 16) || sk[0] % 8 || sk[1] % 8 || sv[0] % 8 || sv[1] % 8)
    return fail("q/k/v need a contiguous head_dim and 16-byte aligned rows");
  bb::SparseDecodeParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.idx = idx;
  p.n_dev = n_dev;
  p.out = static_cast<uint16_t*>(out);
  p.sq = sq; p.sk0 = sk[0]; p.sk1 = sk[1]; p.sv0 = sv[0]; p.sv1 = sv[1];
  if (si) { p.si0 = si[0]; p.si1 = si[1]; }
  p.so = so;
  p.n = n_dev ? cap : (n < cap ? n : cap);
  p.cap = cap;
  p.H = H; p.Hkv = Hkv; p.G = G; p.D = D; p.rows = rows;
  p.front = front; p.window = window; p.route_k = route_k; p.f16 = is_f16 ? 1 : 0;
  const int64_t total = (int64_t)front + window + route_k;
  p.split_len = decode_chunk_len(total, rows, splits, 0);
  p.n_splits = (int)cdiv(total > 0 ? total : 1, p.split_len);
  p.c = (float)((double)scale * 1.4426950408889634);
  const size_t need = bb_sparse_decode_workspace(H, Hkv, D, rows, front, window, route_k, splits);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  p.part = static_cast<float*>(ws);
  return hip_status(bb::launch_sparse_decode(p, static_cast<hipStream_t>(stream)), "bb_sparse_decode");
}

static int64_t route_chunk_len(int64_t cap, int Hkv, int splits) { return decode_chunk_len(cap, Hkv, splits, 256, 4); }

size_t bb_decode_route_workspace(int64_t cap, int H, int Hkv, int splits, int k_route) {
  if (cap <= 0 || H <= 0 || Hkv <= 0 || H % Hkv) return 0;
  const int64_t ns = cdiv(cap, route_chunk_len(cap, Hkv, splits));
  size_t b = align256((size_t)H * cap * 4) + 2 * align256((size_t)Hkv * ns * (H / Hkv) * 4);
  if (k_route > 0) b += align256((size_t)Hkv * cap * 8) + align256(bb::topk_workspace_bytes(cap, Hkv));
  return b;
}

// Decode routing for bb_decode_route and bb_decode_step (app: the step's new row, appended by the scores pass).
static int route_impl(const void* q, int64_t sq, const void* k, const int64_t* sk, int64_t n, const int64_t* n_dev,
                      int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                      float* probs_out, int k_route, int32_t* idx_out, void* ws, size_t ws_bytes,
                      const bb::RowAppend* app, hipStream_t st);

int bb_decode_route(const void* q, int64_t sq, const void* k, const int64_t* sk, int64_t n, const int64_t* n_dev,
                    int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                    float* probs_out, int k_route, int32_t* idx_out, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  return route_impl(q, sq, k, sk, n, n_dev, cap, H, Hkv, D, front, window, scale, splits, is_f16, probs_out, k_route,
                    idx_out, ws, ws_bytes, nullptr, static_cast<hipStream_t>(stream));
}

static int route_impl(const void* q, int64_t sq, const void* k, const int64_t* sk, int64_t n, const int64_t* n_dev,
                      int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                      float* probs_out, int k_route, int32_t* idx_out, void* ws, size_t ws_bytes,
                      const bb::RowAppend* app, hipStream_t st) {
  if (!q || !k || !sk || !probs_out) return fail("q [H,D] and k [Hkv,CAP,D] must match");
  if (H <= 0 || Hkv <= 0 || H % Hkv || cap <= 0) return fail("q [H,D] and k [Hkv,CAP,D] must match");
  const int G = H / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail("decode routing: groups %d unsupported", G);
  if (D != 64 && D != 128) return fail("decode routing: head_dim %d unsupported (64 or 128)", D);
  if (front < 0 || window < 0) return fail("front >= 0 and window >= 0 required");
  if (k_route < 0 || (k_route > 0 && !idx_out)) return fail("decode routing: k_route must be >= 0 with an output");
  if (!(scale > 0.0f)) return fail("scale must be positive");
  if (!aligned(q, 2) || !aligned(k, 16) || sk[0] % 8 || sk[1] % 8)
    return fail("q/k need a contiguous head_dim and 16-byte aligned rows");
  const size_t need = bb_decode_route_workspace(cap, H, Hkv, splits, k_route);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  bb::DecodeRouteParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.n_dev = n_dev;
  p.sq = sq; p.sk0 = sk[0]; p.sk1 = sk[1];
  p.n = n_dev ? cap : (n < cap ? n : cap);
  p.cap = cap;
  p.H = H; p.Hkv = Hkv; p.D = D; p.front = front; p.window = window; p.f16 = is_f16 ? 1 : 0;
  p.split_len = route_chunk_len(cap, Hkv, splits);
  p.n_splits = (int)cdiv(cap, p.split_len);
  p.c = (float)((double)scale * 1.4426950408889634);
  char* w = static_cast<char*>(ws);
  p.scores = reinterpret_cast<float*>(w); w += align256((size_t)H * cap * 4);
  p.stat_m = reinterpret_cast<float*>(w); w += align256((size_t)Hkv * p.n_splits * G * 4);
  p.stat_l = reinterpret_cast<float*>(w); w += align256((size_t)Hkv * p.n_splits * G * 4);
  p.probs = probs_out;
  if (k_route > 0) {
    p.keys = reinterpret_cast<uint64_t*>(w);
    w += align256((size_t)Hkv * cap * 8);
    bb::topk_hist_meta(w, cap, Hkv, &p.top_hist, &p.top_meta);  // filled by the pool pass
  }
  if (app) p.app = *app;
  int rc = hip_status(bb::launch_decode_route_probs(p, st), "bb_decode_route");
  if (rc != BB_OK || k_route == 0) return rc;
  return hip_status(bb::launch_topk_rows(p.keys, Hkv, cap, p.n, n_dev, front, window, k_route, idx_out, w,
                                         bb::topk_workspace_bytes(cap, Hkv), bb::kTopFloatKeys | bb::kTopHistReady, st),
                    "bb_decode_route top-k");
}

int bb_kv_append(void* k, const int64_t* sk, void* v, const int64_t* sv, const void* knew, int64_t sknew,
                 const void* vnew, int64_t svnew, int Hkv, int D, int64_t cap, int64_t* n_dev, int64_t n_inc,
                 void* stream) {
  g_err[0] = 0;
  if (!k || !v || !sk || !sv || !knew || !vnew || !n_dev) return fail("kv_append: null argument");
  if (Hkv <= 0 || D <= 0 || D % 8 || cap <= 0) return fail("kv_append: rows must be whole 16-byte units");
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(knew, 16) || !aligned(vnew, 16) || sk[0] % 8 || sk[1] % 8 ||
      sv[0] % 8 || sv[1] % 8 || sknew % 8 || svnew % 8)
    return fail("kv_append: rows must be 16-byte aligned");
  if (!aligned(n_dev, 8)) return fail("kv_append: misaligned length");
  return hip_status(bb::launch_kv_append(static_cast<uint16_t*>(k), sk[0], sk[1], static_cast<uint16_t*>(v), sv[0],
                                         sv[1], static_cast<const uint16_t*>(knew), sknew,
                                         static_cast<const uint16_t*>(vnew), svnew, Hkv, D, cap, n_dev, n_inc,
                                         static_cast<hipStream_t>(stream)),
                    "bb_kv_append");
}

size_t bb_decode_step_workspace(int64_t cap, int H, int Hkv, int D, int front, int window, int routed) {
  if (cap <= 0 || H <= 0 || Hkv <= 0 || H % Hkv || routed < 0) return 0;
  const int fr = routed > 0 ? front : 0, win = routed > 0 ? window : (int)std::min<int64_t>(cap, 0x7fffffff);
  size_t b = align256(bb_sparse_decode_workspace(H, Hkv, D, Hkv, fr, win, routed, 0));
  if (routed > 0) b += align256((size_t)Hkv * cap * 4) + bb_decode_route_workspace(cap, H, Hkv, 0, routed);
  return b;
}

int bb_decode_step(const void* q, int64_t sq, void* k, const int64_t* sk, void* v, const int64_t* sv, const void* knew,
                   int64_t sknew, const void* vnew, int64_t svnew, int64_t* n_dev, int64_t advance, int64_t cap, int H,
                   int Hkv, int D, int front, int window, int routed, float scale, int is_f16, int32_t* idx_out,
                   void* out, int64_t so, void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (!q || !k || !v || !sk || !sv || !knew || !vnew || !n_dev || !out) return fail("decode step: null argument");
  if (H <= 0 || Hkv <= 0 || H % Hkv || cap <= 0) return fail("q [H,D] and k/v [Hkv,N,D] must match");
  const int G = H / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail("decode: groups %d unsupported", G);
  if (D != 64 && D != 128) return fail("decode: head_dim %d unsupported (64 or 128)", D);
  if (routed < 0 || (routed > 0 && !idx_out)) return fail("decode step: routed must be >= 0 with an index output");
  if (routed > 0 && (front < 0 || window < 0)) return fail("front >= 0 and window >= 0 required");
  if (!(scale > 0.0f)) return fail("scale must be positive");
  if (advance < 0) return fail("decode step: advance must be >= 0");
  if (!aligned(q, 2) || !aligned(k, 16) || !aligned(v, 16) || !aligned(knew, 16) || !aligned(vnew, 16) || sk[0] % 8 ||
      sk[1] % 8 || sv[0] % 8 || sv[1] % 8 || sknew % 8 || svnew % 8)
    return fail("q/k/v need a contiguous head_dim and 16-byte aligned rows");
  if (!aligned(n_dev, 8)) return fail("decode step: misaligned length");
  const size_t need = bb_decode_step_workspace(cap, H, Hkv, D, front, window, routed);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  bb::RowAppend app;
  app.knew = static_cast<const uint16_t*>(knew);
  app.vnew = static_cast<const uint16_t*>(vnew);
  app.k = static_cast<uint16_t*>(k);
  app.v = static_cast<uint16_t*>(v);
  app.skn = sknew; app.svn = svnew; app.sk0 = sk[0]; app.sk1 = sk[1]; app.sv0 = sv[0]; app.sv1 = sv[1];
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* w = static_cast<char*>(ws);
  const int fr = routed > 0 ? front : 0, win = routed > 0 ? window : (int)std::min<int64_t>(cap, 0x7fffffff);
  const size_t part_bytes = bb_sparse_decode_workspace(H, Hkv, D, Hkv, fr, win, routed, 0);
  float* part = reinterpret_cast<float*>(w);
  w += align256(part_bytes);
  const float* route_scores = nullptr;
  if (routed > 0) {  // decode routing appends the row (its scores pass is the first to read the cache)
    float* probs = reinterpret_cast<float*>(w);
    w += align256((size_t)Hkv * cap * 4);
    route_scores = reinterpret_cast<const float*>(w);  // route_impl's first workspace block: scores [H][cap]
    const size_t rws = bb_decode_route_workspace(cap, H, Hkv, 0, routed);
    int rc = route_impl(q, sq, k, sk, cap, n_dev, cap, H, Hkv, D, front, window, scale, 0, is_f16, probs, routed,
                        idx_out, w, rws, &app, st);
    if (rc != BB_OK) return rc;
  }
  bb::SparseDecodeParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.idx = routed > 0 ? idx_out : nullptr;
  p.n_dev = n_dev;
  p.out = static_cast<uint16_t*>(out);
  p.sq = sq; p.sk0 = sk[0]; p.sk1 = sk[1]; p.sv0 = sv[0]; p.sv1 = sv[1];
  p.si0 = routed; p.si1 = 1;
  p.so = so;
  p.n = cap;
  p.cap = cap;
  p.H = H; p.Hkv = Hkv; p.G = G; p.D = D; p.rows = Hkv;
  p.front = fr; p.window = win; p.route_k = routed; p.f16 = is_f16 ? 1 : 0;
  const int64_t total = (int64_t)fr + win + routed;
  p.split_len = decode_chunk_len(total, Hkv, 0, 0);
  p.n_splits = (int)cdiv(total > 0 ? total : 1, p.split_len);
  p.c = (float)((double)scale * 1.4426950408889634);
  p.part = part;
  if (routed == 0) p.app = app;  // dense: the decode kernel is the first to read the cache
  p.n_advance = advance > 0 ? n_dev : nullptr;
  p.advance = advance;
  p.xs = route_scores;  // routed: the decode reuses the routing pass's scores and reads only V rows
  p.xs_stride = cap;
  return hip_status(bb::launch_sparse_decode(p, st), "bb_decode_step");
}

int bb_gather_rows(const void* src, const int64_t* ss, int64_t n_src, int heads, const int64_t* idx, int64_t si0, int m,
                   int D, void* dst, const int64_t* sd, void* stream) {
  g_err[0] = 0;
  if (!src || !ss || !dst || !sd || (m > 0 && !idx)) return fail("gather: null argument");
  if (heads < 0 || m < 0 || D <= 0 || D % 8) return fail("gather: rows must be whole 16-byte units");
  if (!aligned(src, 16) || !aligned(dst, 16) || ss[0] % 8 || ss[1] % 8 || sd[0] % 8 || sd[1] % 8)
    return fail("gather: rows must be 16-byte aligned");
  return hip_status(bb::launch_gather_rows(static_cast<const uint16_t*>(src), ss[0], ss[1], n_src, heads, idx, si0, m, D,
                                           static_cast<uint16_t*>(dst), sd[0], sd[1], static_cast<hipStream_t>(stream)),
                    "bb_gather_rows");
}

size_t bb_topk_f32_workspace(int rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  return align256((size_t)rows * n * 8) + align256(bb::topk_workspace_bytes(n, rows));
}

int bb_topk_f32(const float* vals, int64_t sv0, int rows, int64_t n, int front, int tail, int budget, int32_t* out,
                void* ws, size_t ws_bytes, void* stream) {
  g_err[0] = 0;
  if (!vals || !out) return fail("topk: null argument");
  if (rows <= 0 || n <= 0 || budget <= 0 || front < 0 || tail < 0) return fail("topk: empty selection");
  const size_t need = bb_topk_f32_workspace(rows, n);
  if (!ws || ws_bytes < need) return fail("workspace of %zu bytes required", need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint64_t* keys = static_cast<uint64_t*>(ws);
  int rc = hip_status(bb::launch_f32_keys(vals, sv0, rows, n, keys, st), "bb_topk_f32 keys");
  if (rc != BB_OK) return rc;
  char* w = static_cast<char*>(ws) + align256((size_t)rows * n * 8);
  return hip_status(bb::launch_topk_rows(keys, rows, n, n, nullptr, front, tail, budget, out, w,
                                         bb::topk_workspace_bytes(n, rows), bb::kTopFloatKeys, st),
                    "bb_topk_f32");
}

int bb_rms_norm(const void* x, int64_t sx, int rows, int D, const void* w, float eps, int is_f16, void* out,
                int64_t so, void* stream) {
  g_err[0] = 0;
  if (!x || !w || !out) return fail("rms_norm: null argument");
  if (rows < 0 || D <= 0 || D % 8 || D > 8192) return fail("rms_norm: hidden size %d unsupported", D);
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16) || sx % 8 || so % 8)
    return fail("rms_norm: rows must be 16-byte aligned");
  return hip_status(bb::launch_rms_norm(static_cast<const uint16_t*>(x), sx, nullptr, 0, rows, D,
                                        static_cast<const uint16_t*>(w), eps, is_f16 ? 1 : 0,
                                        static_cast<uint16_t*>(out), so, nullptr, 0, static_cast<hipStream_t>(stream)),
                    "bb_rms_norm");
}

int bb_add_rms_norm(const void* x, int64_t sx, const void* res, int64_t sr, int rows, int D, const void* w, float eps,
                    int is_f16, void* sum, int64_t ssum, void* out, int64_t so, void* stream) {
  g_err[0] = 0;
  if (!x || !res || !w || !sum || !out) return fail("add_rms_norm: null argument");
  if (rows < 0 || D <= 0 || D % 8 || D > 8192) return fail("add_rms_norm: hidden size %d unsupported", D);
  if (!aligned(x, 16) || !aligned(res, 16) || !aligned(w, 16) || !aligned(sum, 16) || !aligned(out, 16) || sx % 8 ||
      sr % 8 || ssum % 8 || so % 8)
    return fail("add_rms_norm: rows must be 16-byte aligned");
  return hip_status(bb::launch_rms_norm(static_cast<const uint16_t*>(x), sx, static_cast<const uint16_t*>(res), sr,
                                        rows, D, static_cast<const uint16_t*>(w), eps, is_f16 ? 1 : 0,
                                        static_cast<uint16_t*>(out), so, static_cast<uint16_t*>(sum), ssum,
                                        static_cast<hipStream_t>(stream)),
                    "bb_add_rms_norm");
}

int bb_gemv(const void* w, int64_t sw, int N, int K, const void* x, int glu, int is_f16, void* y, void* stream) {
  g_err[0] = 0;
  if (!w || !x || !y) return fail("gemv: null argument");
  if (N < 0 || K <= 0 || K % 8 || K > 16384) return fail("gemv: K = %d must be a positive multiple of 8, at most 16384", K);
  if (!aligned(w, 16) || !aligned(x, 16) || sw % 8 || sw < K || !aligned(y, 2))
    return fail("gemv: W rows and x must be 16-byte aligned");
  return hip_status(bb::launch_gemv(static_cast<const uint16_t*>(w), sw, N, K, static_cast<const uint16_t*>(x), nullptr,
                                    glu != 0, is_f16 ? 1 : 0, static_cast<uint16_t*>(y),
                                    static_cast<hipStream_t>(stream)),
                    "bb_gemv");
}

int bb_gemv_norm(const void* w, int64_t sw, int N, int K, const void* x, const void* res, const void* norm_w,
                 float eps, int glu, int is_f16, void* sum, void* y, void* stream) {
  g_err[0] = 0;
  if (!w || !x || !norm_w || !y || (res != nullptr) != (sum != nullptr)) return fail("gemv_norm: null argument");
  if (N < 0 || K <= 0 || K % 8 || K > 8192)
    return fail("gemv_norm: K = %d must be a positive multiple of 8, at most 8192", K);
  if (!aligned(w, 16) || !aligned(x, 16) || !aligned(norm_w, 16) || (res && (!aligned(res, 16) || !aligned(sum, 16))) ||
      sw % 8 || sw < K || !aligned(y, 2))
    return fail("gemv_norm: W rows, x, res, sum and the norm weight must be 16-byte aligned");
  const bb::GemvNorm nm{static_cast<const uint16_t*>(res), static_cast<const uint16_t*>(norm_w), eps,
                        static_cast<uint16_t*>(sum)};
  return hip_status(bb::launch_gemv(static_cast<const uint16_t*>(w), sw, N, K, static_cast<const uint16_t*>(x), &nm,
                                    glu != 0, is_f16 ? 1 : 0, static_cast<uint16_t*>(y),
                                    static_cast<hipStream_t>(stream)),
                    "bb_gemv_norm");
}

int bb_silu_mul(const void* g, const void* u, int64_t n, int is_f16, void* out, void* stream) {
  g_err[0] = 0;
  if (!g || !u || !out) return fail("silu_mul: null argument");
  if (n < 0 || n % 8) return fail("silu_mul: length %lld must be a multiple of 8", (long long)n);
  if (!aligned(g, 16) || !aligned(u, 16) || !aligned(out, 16)) return fail("silu_mul: buffers must be 16-byte aligned");
  return hip_status(bb::launch_silu_mul(static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u), n,
                                        is_f16 ? 1 : 0, static_cast<uint16_t*>(out), static_cast<hipStream_t>(stream)),
                    "bb_silu_mul");
}

int bb_argmax(const void* x, int64_t n, int dtype, int64_t* out, void* stream) {
  g_err[0] = 0;
  if (!x || !out) return fail("argmax: null argument");
  if (n <= 0 || n > 0x7ffffffe) return fail("argmax: row length %lld out of range", (long long)n);
  if (dtype < 0 || dtype > 2) return fail("argmax: dtype must be 0 (fp32), 1 (bf16) or 2 (fp16)");
  return hip_status(bb::launch_argmax(x, n, dtype, aligned(x, 16), out, static_cast<hipStream_t>(stream)), "bb_argmax");
}

int bb_stream_read(const void* buf, size_t bytes, uint32_t* sink, int workgroups, void* stream) {
  g_err[0] = 0;
  if (!buf || !sink) return fail("stream_read: null argument");
  if (bytes % 16 || !aligned(buf, 16) || workgroups <= 0) return fail("stream_read: 16-byte aligned whole units");
  return hip_status(bb::launch_stream_read(buf, (int64_t)bytes, sink, workgroups, static_cast<hipStream_t>(stream)),
                    "bb_stream_read");
}

int bb_rope_inplace(void* x, const int64_t* sx, int B, int Hh, int64_t T, int D, const void* cos, const void* sin,
                    const int64_t* sc, int is_f16, void* stream) {
  g_err[0] = 0;
  if (!x || !cos || !sin || !sx || !sc) return fail("rope: null argument");
  if (D % 16) return fail("rope: head_dim must be a multiple of 16");
  if (!aligned(x, 16) || !aligned(cos, 16) || !aligned(sin, 16) || sx[0] % 8 || sx[1] % 8 || sx[2] % 8 || sc[0] % 8 ||
      sc[1] % 8)
    return fail("rope: rows must be 16-byte aligned");
  return hip_status(bb::launch_rope(static_cast<uint16_t*>(x), sx[0], sx[1], sx[2], B, Hh, T, D,
                                    static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), sc[0], sc[1],
                                    is_f16 ? 1 : 0, static_cast<hipStream_t>(stream)),
                    "bb_rope_inplace");
}

}  // extern "C"
