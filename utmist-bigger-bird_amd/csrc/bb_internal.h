// Host-side launch descriptors shared between the kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bb {

// Sparse flash attention (one joint softmax over front | causal window | routed keys).
struct FlashParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* vt;       // V^T [n_kvbh][D][np] (keys >= N zero)
  const int32_t* idx;       // [BH, n_groups, route_k] (strided), -1 = empty slot
  const uint8_t* key_mask;  // [B, N] bool (strided by smb), or null
  uint16_t* out;            // [BH, T, D] view (strided)
  float* part_o;            // split mode: [n_chunks][BH][T][D]
  float* part_ml;           // split mode: [n_chunks][BH][T][2] (running max in log2 units, denominator)
  int64_t sq0, sq1, sk0, sk1, sv0, sv1, si0, si1, si2, smb, so0, so1;
  int64_t N, T, offset, row_end, route_chunk, key_chunk, np;
  int64_t pos_step;         // absolute position of query row t = offset + t * pos_step (0: every row at offset)
  const uint16_t* rtiles;   // pre-gathered routed tiles [BH][n_groups][rt_batches][K tile | V^T tile], or null
  int rt_batches;           // 64-slot batches of one route list (route_k rounded up to 64)
  int f16;                  // 16-bit element type: 0 bf16, 1 fp16
  int BH, H, G, Hkv_pb, n_kvbh, front, window, route_k, n_groups;
  int row_tiles, head_splits, n_chunks, remap;
  float c;  // scale * log2(e)
};

hipError_t launch_flash(const FlashParams& p, int D, int hpw, bool split, hipStream_t stream);
hipError_t launch_flash_merge(const FlashParams& p, int D, hipStream_t stream);
// Software-pipelined main-pass kernel (head_dim 128, kv_groups % 4 == 0, no token mask, 64-aligned route groups).
// The pipelined kernel with hpw query heads per workgroup (4, 2 or 1; the schedule's rows per tile 32 x 8 / hpw).
bool flash_pipe_supported(const FlashParams& p, int D, int hpw);
hipError_t launch_flash_pipe(const FlashParams& p, int hpw, hipStream_t stream);
// Bytes of the pre-gathered routed tiles of one call, and the kernel that writes them (p.rtiles) for the main pass.
size_t route_tiles_bytes(int BH, int n_groups, int route_k);
hipError_t launch_route_tiles(const FlashParams& p, uint16_t* rt, hipStream_t stream);
hipError_t launch_transpose_v(const uint16_t* v, int64_t sv0, int64_t sv1, int n_kvbh, int64_t N, int64_t np, int D,
                              uint16_t* vt, hipStream_t stream);

// Routing (pooled softmax of the route queries, then per-head top-k).
struct RoutesParams {
  const uint16_t* q;  // [BH, n, D] strided (sq0 head, sq1 token)
  const uint16_t* k;  // [BKV, n, D] strided
  const int64_t* qpos;  // [r]
  int64_t sq0, sq1, sk0, sk1;
  int64_t n;
  int H, Hkv, B, D, r, sink, window, budget, pool_max;
  int scores_reference_order;  // 1: every score by the reference-order chain (no MFMA), for cross-checks
  int f16;              // q and k are fp16 (scores in torch's CPU fp16 order, stored as fp16); else bf16
  float scaling;
  uint16_t* scores;     // [B*Hkv][G*r][n] bf16 workspace
  uint32_t* rowmax;     // [B*H*r] row maxima (fp32 bits)
  uint64_t* rowsum;     // [B*H*r] fixed point 2^40
  uint64_t* pooled;     // [B*H][pstride] fixed point 2^40
  int32_t* out_idx;     // [B*H][budget]
  int64_t pstride;      // row stride of pooled (n for prefill routes)
  const int64_t* n_dev; // top-k range length from device memory (decode routing), or null
  int float_keys;       // top-k keys are fp32 bits of positive values (binned by value, not by bit length)
};

size_t routes_workspace_bytes(int64_t n, int H, int Hkv, int B, int r);
hipError_t launch_routes(RoutesParams& p, void* ws, size_t ws_bytes, hipStream_t stream);

// INT8 KV cache.
// With x1 set, a second input of the same shape and strides goes to (q1, scale1) in the same launch.
// Element kinds: 0 bf16, 1 fp32, 2 fp16 (quantise input, dequantise output).
hipError_t launch_int8_quantize(const void* x, int x_kind, int64_t rows, int64_t row_stride, int inner, int64_t inner_stride,
                                int D, float min_scale, int8_t* q, void* scale, int scale_is_f16, hipStream_t stream,
                                const void* x1 = nullptr, int8_t* q1 = nullptr, void* scale1 = nullptr);
hipError_t launch_int8_dequantize(const int8_t* q, const void* scale, int scale_is_f16, int64_t rows, int D,
                                  void* out, int out_kind, hipStream_t stream);

struct DecodeParams {
  const uint16_t* q;   // [B*H, D] (row stride sq)
  const int8_t* k8;    // [cap, Hkv, D] token-major
  const int8_t* v8;
  const void* ks;      // [cap, Hkv] fp16 or fp32
  const void* vs;
  const uint16_t* kb;  // bf16 cache variant: [Hkv, cap, D] (strided) -- used when k8 == null
  const uint16_t* vb;
  int64_t sq, skb0, skb1, svb0, svb1;
  int64_t n;
  int H, Hkv, D, scale_is_f16, n_splits;
  int64_t split_len;
  float c;             // scale * log2(e)
  uint16_t* out;       // [H, D]
  int64_t so;
  float* part;         // [H][n_splits][D + 2]
  // Optional: the step's new token. Its K and V rows (bf16 [Hkv, D], head strides sknew / svnew) are quantised into
  // cache row n - 1 (wk8 / wv8 with scales wks / wvs, the same buffers as k8 / v8 / ks / vs) before they are read.
  const uint16_t* knew;
  const uint16_t* vnew;
  int64_t sknew, svnew;
  float min_scale;
  int8_t* wk8;
  int8_t* wv8;
  void* wks;
  void* wvs;
};
size_t decode_workspace_bytes(int H, int D, int n_splits);
// Whether launch_decode quantises the new rows (knew / vnew) inside the decode kernel; otherwise the caller quantises
// them first and passes knew = nullptr.
bool decode_fuses_append(const DecodeParams& p);
hipError_t launch_decode(const DecodeParams& p, hipStream_t stream);

// A decode step's new K / V row folded into the first kernel that reads the cache: the row at position n - 1 (n the
// current length, which already counts it) is read from knew / vnew instead of the cache, and the lanes that read it
// also write it to the cache rows (k, v), so that later kernels find it there. Only when 1 <= n <= cap; knew = null
// switches it off.
struct RowAppend {
  const uint16_t* knew;  // [Hkv, D] (head stride skn)
  const uint16_t* vnew;  // [Hkv, D] (head stride svn)
  uint16_t* k;           // the cache [Hkv, cap, D] (strides sk0 head, sk1 token), writable
  uint16_t* v;           // (strides sv0, sv1)
  int64_t skn, svn, sk0, sk1, sv0, sv1;
};

// Split-K sparse decode over a bf16 / fp16 KV cache (front | window | routed keys per route row).
struct SparseDecodeParams {
  const uint16_t* q;     // [H, D] (row stride sq)
  const uint16_t* k;     // [Hkv, cap, D] strided (sk0 head, sk1 token)
  const uint16_t* v;
  const int32_t* idx;    // [rows, route_k] strided (si0, si1), -1 = empty
  const int64_t* n_dev;  // current length in device memory, or null (then n)
  uint16_t* out;         // [H, D] (row stride so)
  float* part;           // [H][n_splits][D + 2]
  int64_t sq, sk0, sk1, sv0, sv1, si0, si1, so;
  int64_t n, cap, split_len;
  int H, Hkv, G, D, rows, front, window, route_k, n_splits, f16;
  float c;               // scale * log2(e)
  RowAppend app;         // the step's new row (dense decode without routing), or app.knew = null
  int64_t* n_advance;    // after the merge: *n_advance += advance when the row was appended (n_advance = n_dev), or null
  int64_t advance;
  const float* xs;       // scores of this query from decode routing ([H][xs_stride], scale * log2(e) applied), or null
  int64_t xs_stride;
};
hipError_t launch_sparse_decode(const SparseDecodeParams& p, hipStream_t stream);

// Decode routing: pooled probabilities over the cached keys for one query token.
struct DecodeRouteParams {
  const uint16_t* q;     // [H, D] (row stride sq)
  const uint16_t* k;     // [Hkv, cap, D] strided
  const int64_t* n_dev;
  float* scores;         // [H, cap] workspace (log2 units)
  float* stat_m;         // [Hkv][n_splits][G]
  float* stat_l;
  float* probs;          // [Hkv, cap] output
  uint64_t* keys;        // [Hkv, cap] top-k keys, or null
  uint32_t* top_hist;    // [Hkv][top-k bins] histogram filled while the keys are written (with keys), or null
  uint32_t* top_meta;    // [Hkv][8] top-k counters, cleared by the scores pass when top_hist is set
  int64_t sq, sk0, sk1;
  int64_t n, cap, split_len;
  int H, Hkv, D, front, window, n_splits, f16;
  float c;
  RowAppend app;         // the step's new row (the scores pass appends it), or app.knew = null
};
hipError_t launch_decode_route_probs(const DecodeRouteParams& p, hipStream_t stream);
// Top-`budget` of 64-bit keys per row over [front, n - window) (n from n_dev when set), ascending int32 indices;
// rows of `stride` keys; the workspace comes from topk_workspace_bytes. Flags: kTopFloatKeys when the keys are fp32
// bits of positive values (0 for the rest), kTopHistReady when the histogram and counters in the workspace
// (topk_hist_meta) were already filled and cleared by the producer of the keys.
constexpr int kTopFloatKeys = 1, kTopHistReady = 2;
size_t topk_workspace_bytes(int64_t stride, int rows);
void topk_hist_meta(void* ws, int64_t stride, int rows, uint32_t** hist, uint32_t** meta);
hipError_t launch_topk_rows(const uint64_t* keys, int rows, int64_t stride, int64_t n, const int64_t* n_dev,
                            int front, int window, int budget, int32_t* out, void* ws, size_t ws_bytes, int flags,
                            hipStream_t stream);

// Row gather (cache compaction) and float -> top-k key conversion.
hipError_t launch_gather_rows(const uint16_t* src, int64_t ss0, int64_t ss1, int64_t n_src, int heads,
                              const int64_t* idx, int64_t si0, int m, int D, uint16_t* dst, int64_t sd0, int64_t sd1,
                              hipStream_t stream);
// HF LlamaRMSNorm arithmetic on rows of a 16-bit tensor (D % 8 == 0, D <= 8192).
// (res, sum both null, or both set: x + res is normalised and written to sum)
hipError_t launch_rms_norm(const uint16_t* x, int64_t sx, const uint16_t* res, int64_t sr, int rows, int D,
                           const uint16_t* w, float eps, int f16, uint16_t* out, int64_t so, uint16_t* sum,
                           int64_t ssum, hipStream_t stream);
// The RMSNorm that a GEMV applies to its input row first (x + res when res is set; the sum goes to `sum`).
struct GemvNorm {
  const uint16_t* res;  // residual added before the norm, or null
  const uint16_t* w;    // the norm's weight [K]
  float eps;
  uint16_t* sum;        // x + res [K] (with res; must not overlap x or res)
};
// y[N] = W[N, K] x[K] for one token (16-bit, row stride sw; K % 8 == 0, K <= 16384; 16-byte aligned rows and x);
// nm: x replaced by its RMSNorm (K <= 8192); glu: W has 2N rows (gate over up) and y = round(round(silu(g)) u).
hipError_t launch_gemv(const uint16_t* w, int64_t sw, int N, int K, const uint16_t* x, const GemvNorm* nm, bool glu,
                       int f16, uint16_t* y, hipStream_t stream);
// out = round(round(silu(g)) u) over n values (n % 8 == 0, 16-byte aligned).
hipError_t launch_silu_mul(const uint16_t* g, const uint16_t* u, int64_t n, int f16, uint16_t* out,
                           hipStream_t stream);
// Index of the largest element of x [n] (kind 0 fp32, 1 bf16, 2 fp16; vec16: 16-byte aligned), to out[0].
// Decode-step cache append at a device-side length (advanced by n_inc afterwards).
hipError_t launch_kv_append(uint16_t* k, int64_t sk0, int64_t sk1, uint16_t* v, int64_t sv0, int64_t sv1,
                            const uint16_t* knew, int64_t skn, const uint16_t* vnew, int64_t svn, int heads, int D,
                            int64_t cap, int64_t* n_dev, int64_t n_inc, hipStream_t stream);
hipError_t launch_argmax(const void* x, int64_t n, int kind, bool vec16, int64_t* out, hipStream_t stream);
hipError_t launch_f32_keys(const float* vals, int64_t sv0, int rows, int64_t n, uint64_t* keys, hipStream_t stream);

// RoPE in place (HF apply_rotary_pos_emb arithmetic in bf16, or fp16 when f16).
hipError_t launch_rope(uint16_t* x, int64_t sx0, int64_t sx1, int64_t sx2, int B, int Hh, int64_t T, int D,
                       const uint16_t* cos, const uint16_t* sin, int64_t sc0, int64_t sc1, int f16, hipStream_t stream);

// HBM read ceiling probe (bb_probe.hip): XOR of `bytes` (a multiple of 16) of buf, one word per workgroup to sink.
hipError_t launch_stream_read(const void* buf, int64_t bytes, uint32_t* sink, int workgroups, hipStream_t stream);

}  // namespace bb
