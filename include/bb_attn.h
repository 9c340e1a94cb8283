/*
 * bb_attn -- C ABI of the MI355X-native Bigger Bird v3 sparse prefill path (gfx950 HIP kernels).
 *
 * Conventions
 *   - Every tensor argument is a device pointer plus element strides (int64); the innermost (head_dim) stride is 1.
 *     bf16 tensors are passed as raw 16-bit storage.
 *   - All launches are asynchronous on `stream` (a hipStream_t; NULL = the null stream). Nothing synchronises the
 *     host, nothing allocates or frees device memory: callers pass any workspace the *_workspace() query asks for.
 *   - Return value: 0 on success; BB_EINVAL (-1) for an argument error, whose message (bb_last_error()) matches the
 *     reference's ValueError text where the reference raises one; BB_EHIP (-2) when a HIP launch fails.
 *   - Functions are re-entrant; bb_last_error() is per host thread.
 */
#ifndef BB_ATTN_H
#define BB_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BB_OK 0
#define BB_EINVAL (-1)
#define BB_EHIP (-2)

/* Library version (major * 10000 + minor * 100 + patch). The minor number changes with every change of an entry
 * point's parameter list, so a caller built against another header can refuse the library:
 *   100  first release
 *   200  bb_sparse_flash and bb_routes take is_f16 (after D); bb_sparse_flash_workspace takes n_groups (after
 *        route_k) and has_key_mask (last); bb_rope_inplace takes is_f16 (before stream); bb_init and bb_stream_read
 *        added
 *   201  bb_decode_step and bb_decode_step_workspace added
 *   202  bb_int8_quantize / bb_int8_quantize_pair take an element kind (0 bf16, 1 fp32, 2 fp16) where they took
 *        x_is_f32, and bb_int8_dequantize an output kind where it took out_is_f32 (the old values keep their
 *        meaning)
 *   203  bb_add_rms_norm, bb_silu_mul, bb_gemv and bb_gemv_norm added */
#define BB_ABI_VERSION 203
int bb_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* bb_last_error(void);

/* Optional set-up for the current device (no reference counterpart): resolves the device address of
 * bb_decode_noalloc's static scratch, which that entry point otherwise looks up on its first call on a device. Call
 * it once per device before capturing bb_decode_noalloc into a HIP graph. Allocates nothing. */
int bb_init(void);

/*
 * Sparse flash attention: one joint softmax over front anchors | causal local window | routed keys.
 * Replaces bigger_bird_flash(q, k, v, indices, front=, window=, token_mask=, num_heads=, route_chunk=, kv_groups=,
 * scale=) of kernels/bigger_bird_flash.py:99-138 (and its dispatch at modal_rd/attention.py:41-45).
 *   q    [BH, T, D]   strides sq[3]          k, v [BH / kv_groups, N, D]   strides sk[3], sv[3]
 *   idx  [BH, n_groups, route_k] int32 (-1 = empty), strides si[3]; may be NULL when route_k == 0
 *   key_mask [B, N] uint8 (B = BH / num_heads, row stride smb) or NULL        (token_mask)
 *   out  [BH, T, D]   strides so[3]          (e.g. a permuted view of a [T, BH, D] buffer)
 *   Query row t sits at absolute position t + N - T. Rows >= row_end are not written (row_end = T for all rows).
 *   D in {32, 64, 128}; 16-bit elements: bf16 (is_f16 = 0) or fp16 (is_f16 = 1) for q, k, v, V^T and out alike
 *   (fp32 accumulation and softmax either way); scale > 0.
 *   vt   optional V^T from bb_transpose_v (NULL: transposed into the workspace).
 *   ws/ws_bytes: workspace of at least bb_sparse_flash_workspace(...) bytes (V^T unless given, plus the (O, m, l)
 *   partials of the split-key schedule used for long windows without routes).
 */
int bb_sparse_flash(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                    const int64_t* sv, const void* vt, const int32_t* idx, const int64_t* si, int n_groups,
                    int route_k, const uint8_t* key_mask, int64_t smb, void* out, const int64_t* so, int BH, int64_t T,
                    int64_t N, int D, int is_f16, int num_heads, int kv_groups, int64_t front, int64_t window,
                    int64_t route_chunk, float scale, int64_t row_end, void* ws, size_t ws_bytes, void* stream);

/* Workspace bytes for bb_sparse_flash (n_groups and route_k as passed to it); have_vt != 0 when the caller passes a
 * precomputed V^T, has_key_mask != 0 when it passes a key_mask. Besides V^T and the split partials it holds the
 * routed K/V^T tiles pre-gathered per query head (32 KB per 64 route slots per head) for head_dim 128 with a single
 * route group and no key mask; with several route groups the kernel gathers the routed rows itself (or, with fewer
 * than 4 query heads per KV head, the generic kernel runs) and no tiles are reserved. */
size_t bb_sparse_flash_workspace(int BH, int64_t T, int64_t N, int D, int num_heads, int kv_groups, int64_t front,
                                 int64_t window, int route_k, int n_groups, int64_t row_end, int have_vt,
                                 int has_key_mask);

/*
 * Non-causal exact attention: every one of the T query rows attends all N keys (T <= N), in one launch (plus a merge
 * launch when the keys are split over workgroups). Replaces F.scaled_dot_product_attention(q, k, v,
 * is_causal=False, enable_gqa=True) of RDAttention.exact_attention for 1 < t < n (modal_rd/attention.py:140-141).
 * Arguments as bb_sparse_flash (same layouts, alignment rules, V^T and workspace); bb_exact_attention_workspace
 * sizes the workspace.
 */
int bb_exact_attention(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const void* v,
                       const int64_t* sv, const void* vt, void* out, const int64_t* so, int BH, int64_t T, int64_t N,
                       int D, int is_f16, int num_heads, int kv_groups, float scale, void* ws, size_t ws_bytes,
                       void* stream);
size_t bb_exact_attention_workspace(int BH, int64_t T, int64_t N, int D, int num_heads, int kv_groups, int have_vt);

/*
 * V [n_kvbh, N, D] (strides sv[3]) -> V^T [n_kvbh, D, bb_transpose_v_cols(N)] with zero columns past N: the layout
 * the window tiles stream from. A caller making several bb_sparse_flash calls over the same V (prefill main pass
 * and exact tail) transposes once and passes the result as `vt`. No reference counterpart (the reference's Triton
 * kernel reads V in place).
 */
int bb_transpose_v(const void* v, const int64_t* sv, int n_kvbh, int64_t N, int D, void* vt, void* stream);
int64_t bb_transpose_v_cols(int64_t N);

/*
 * Routing: per query head, the `budget` key columns with the largest mean (pool_max = 0) or max (pool_max = 1)
 * softmax probability over the r route queries at positions qpos, among columns [sink, n - window); returned
 * ascending as int32 in idx_out [B*H, budget]. Replaces RDAttention.routes (modal_rd/attention.py:143-174).
 *   q [B*H, n, D] (strides sq[2]: head, token), k [B*Hkv, n, D] (strides sk[2]); qpos [r] int64 on the device.
 *   pooled_out: optional [B*H, n] uint64 copy of the pooled scores in units of 2^-40 (NULL to skip).
 *   q and k are bf16 (is_f16 = 0) or fp16 (is_f16 = 1), as the reference's routes() runs in the model dtype.
 *   Arithmetic is deterministic: scores rounded from fp32 sums in the accumulation order of the reference's CPU
 *   matmul (bf16: oneDNN AMX-BF16, per 32-element block of d even and odd fp32 chains, rounded to bf16; fp16: one
 *   sequential fp32 chain over d, rounded to fp16), fixed-point softmax sums; results are identical on every run.
 */
int bb_routes(const void* q, const int64_t* sq, const void* k, const int64_t* sk, const int64_t* qpos, int r,
              int B, int H, int Hkv, int64_t n, int D, int is_f16, int64_t sink, int64_t window, int budget,
              float scaling, int pool_max, int32_t* idx_out, uint64_t* pooled_out, void* ws, size_t ws_bytes,
              void* stream);

size_t bb_routes_workspace(int64_t n, int H, int Hkv, int B, int r);

/*
 * Per-row symmetric int8 quantisation of rows (outer, inner) at x + outer*row_stride + inner*inner_stride,
 * D contiguous elements each (x_kind: 0 bf16, 1 fp32, 2 fp16), written token-major: q [outer*inner, D],
 * scale [outer*inner] (fp16 or fp32). Replaces modal_rd/kv_int8.py:19-22 / kernels/kv_int8_triton.py:36-51 (which
 * quantise whatever float dtype the model runs in).
 */
int bb_int8_quantize(const void* x, int x_kind, int64_t outer, int64_t row_stride, int inner, int64_t inner_stride,
                     int D, float min_scale, int8_t* q, void* scale, int scale_is_f16, void* stream);

/* q [rows, D] int8 * scale [rows] in fp32 -> out [rows, D] (out_kind: 0 bf16, 1 fp32, 2 fp16; 16-bit outputs
 * rounded to nearest even). Replaces modal_rd/kv_int8.py:25-26. */
/*
 * bb_int8_quantize of a decode step's new K rows and V rows in one launch: xk and xv share the shape and strides,
 * results to (qk, sk) and (qv, sv). Replaces the per-tensor quantize loop of Int8KVLayer.update
 * (modal_rd/kv_int8.py:107-111).
 */
int bb_int8_quantize_pair(const void* xk, const void* xv, int x_kind, int64_t outer, int64_t row_stride, int inner,
                          int64_t inner_stride, int D, float min_scale, int8_t* qk, void* sk, int8_t* qv, void* sv,
                          int scale_is_f16, void* stream);
int bb_int8_dequantize(const int8_t* q, const void* scale, int scale_is_f16, int64_t rows, int D, void* out,
                       int out_kind, void* stream);

/*
 * Exact attention of one decode token over the first n rows of a KV cache: out [H, D] bf16 from q [H, D] bf16.
 * int8 cache: k8/v8 [cap, Hkv, D] token-major with scales ks/vs [cap, Hkv] (fp16 if scale_is_f16 else fp32).
 * bf16 cache (k8 == NULL): kb/vb [Hkv, cap, D] with strides skb[2], svb[2] (head, token).
 * Replaces RDAttention.exact_attention (modal_rd/attention.py:137-141) over Int8KVLayer's dequantised cache.
 */
int bb_decode(const void* q, int64_t sq, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
              int scale_is_f16, const void* kb, const int64_t* skb, const void* vb, const int64_t* svb, int64_t n,
              int H, int Hkv, int D, float scale, void* out, int64_t so, void* ws, size_t ws_bytes, void* stream);

size_t bb_decode_workspace(int64_t n, int H, int Hkv, int D);

/*
 * One INT8 decode step: quantises the new token's K and V rows (bf16 [Hkv, D], head strides sknew / svnew) into row
 * n - 1 of the int8 cache (k8 / v8 with scales ks / vs, as bb_int8_quantize with min_scale), then attends the query
 * to all n rows, as bb_decode. Replaces the pair Int8KVLayer.update of a one-token step (modal_rd/kv_int8.py:104-112,
 * the new rows quantised into spare capacity) and RDAttention.exact_attention over the cache
 * (modal_rd/attention.py:137-141). For D = 128 with 4 query heads per KV head the decode kernel quantises the rows
 * itself (the workgroup that reads row n - 1 writes it first); other shapes take a quantise launch first. Workspace:
 * bb_decode_workspace(n, ...).
 */
int bb_decode_append(const void* q, int64_t sq, int8_t* k8, void* ks, int8_t* v8, void* vs, int scale_is_f16,
                     const void* knew, int64_t sknew, const void* vnew, int64_t svnew, float min_scale, int64_t n,
                     int H, int Hkv, int D, float scale, void* out, int64_t so, void* ws, size_t ws_bytes,
                     void* stream);

/*
 * bb_decode without a workspace argument and without any allocation: the split partials go to a static device array
 * of bb_decode_noalloc_max_bytes() bytes (2 MiB) inside the library, one per GPU, held until the process ends. No
 * counterpart in the reference: this is for callers that cannot allocate (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Same arguments, kernels and results as bb_decode; a call whose partials
 * (H * splits * (D + 2) * 4 bytes, see bb_decode_workspace) exceed the array returns BB_EINVAL. The array of the
 * current device is used, so `stream` must belong to the current device. Calls that overlap on one GPU (two
 * streams, or two host threads) share the array and race; calls ordered on one stream are safe.
 */
int bb_decode_noalloc(const void* q, int64_t sq, const int8_t* k8, const void* ks, const int8_t* v8, const void* vs,
                      int scale_is_f16, const void* kb, const int64_t* skb, const void* vb, const int64_t* svb,
                      int64_t n, int H, int Hkv, int D, float scale, void* out, int64_t so, void* stream);
size_t bb_decode_noalloc_max_bytes(void);

/*
 * Split-K sparse decode of one query token over a bf16 (is_f16 = 0) or fp16 KV cache. Every route row attends its
 * virtual key list front | window | routed: position j for j < front, n - window + i for the window, idx[row][i]
 * for the routed keys; positions outside [0, n) are skipped. Replaces bigger_bird_decode
 * (kernels/bigger_bird_decode.py:66-108).
 *   q [H, D] (row stride sq); k, v [Hkv, cap, D] (strides sk[2], sv[2]: head, token; any cache view)
 *   idx [rows, route_k] int32 (strides si[2]; -1 = empty): rows = Hkv (pooled: the groups query heads of a KV head
 *   share one list) or rows = H (per-head lists); NULL when route_k == 0
 *   n_dev: the current length as one int64 in device memory (a captured graph stays valid as it grows), or NULL
 *   to use n; splits: key chunks (0 = about four workgroups per CU); out [H, D] (row stride so), input dtype.
 */
int bb_sparse_decode(const void* q, int64_t sq, const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                     const int32_t* idx, const int64_t* si, int rows, int route_k, int64_t n, const int64_t* n_dev,
                     int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                     void* out, int64_t so, void* ws, size_t ws_bytes, void* stream);

size_t bb_sparse_decode_workspace(int H, int Hkv, int D, int rows, int front, int window, int route_k, int splits);

/*
 * Fused decode routing for one query token: probs_out [Hkv, cap] fp32 = per KV head the mean over its query heads
 * of the softmax probability over the first n cached keys, -1 outside [front, n - window); with k_route > 0 also
 * idx_out [Hkv, k_route], the keys with the largest pooled probability (ties to the lower index), ascending, -1 past
 * the eligible count. n / n_dev as in bb_sparse_decode. Replaces pooled_probs and bigger_bird_route
 * (kernels/bigger_bird_route.py:83-115).
 */
int bb_decode_route(const void* q, int64_t sq, const void* k, const int64_t* sk, int64_t n, const int64_t* n_dev,
                    int64_t cap, int H, int Hkv, int D, int front, int window, float scale, int splits, int is_f16,
                    float* probs_out, int k_route, int32_t* idx_out, void* ws, size_t ws_bytes, void* stream);

size_t bb_decode_route_workspace(int64_t cap, int H, int Hkv, int splits, int k_route);

/*
 * One decode step's cache append at a length held in device memory (so a captured graph stays valid as the cache
 * grows): with n = *n_dev, k[h, n, :] = knew[h, :] and v[h, n, :] = vnew[h, :] for the Hkv heads (16-bit elements,
 * D % 8 == 0; k / v strides sk[2] / sv[2]: head, token; knew / vnew head strides), then *n_dev += n_inc. A length
 * outside [0, cap) writes nothing and leaves *n_dev unchanged. One launch in place of the two index_copy_ calls and
 * the length add of a decode step (modal_rd/graph_decode.py's cache append, kernels/bigger_bird_decode.py's callers).
 */
int bb_kv_append(void* k, const int64_t* sk, void* v, const int64_t* sv, const void* knew, int64_t sknew,
                 const void* vnew, int64_t svnew, int Hkv, int D, int64_t cap, int64_t* n_dev, int64_t n_inc,
                 void* stream);

/*
 * One whole decode step over a bf16 / fp16 cache whose length n = *n_dev already counts the step's new row: the new
 * K / V rows (knew / vnew, as in bb_kv_append) become row n - 1 of every KV head (when 1 <= n <= cap), the step
 * attends (routed > 0: pooled decode routing of the top `routed` keys per KV head outside front and the last
 * `window` keys, indices to idx_out [Hkv, routed], then the sparse decode over front | window | routed; routed = 0:
 * dense decode over all n rows, front and window ignored), and afterwards *n_dev += advance when the row was
 * appended. Results are bit-identical to bb_kv_append (at n - 1, n_inc 0) followed by bb_decode_route and
 * bb_sparse_decode (or bb_sparse_decode with front 0 and window cap), with default splits, and the length add; the
 * append and the add ride in the kernels that first read the cache and that end the step, so the step is two
 * launches fewer (the two index_copy_ calls and the length add of modal_rd/graph_decode.py's step, followed by
 * kernels/bigger_bird_route.py:83-115 and kernels/bigger_bird_decode.py:66-108). Workspace from
 * bb_decode_step_workspace.
 */
int bb_decode_step(const void* q, int64_t sq, void* k, const int64_t* sk, void* v, const int64_t* sv, const void* knew,
                   int64_t sknew, const void* vnew, int64_t svnew, int64_t* n_dev, int64_t advance, int64_t cap, int H,
                   int Hkv, int D, int front, int window, int routed, float scale, int is_f16, int32_t* idx_out,
                   void* out, int64_t so, void* ws, size_t ws_bytes, void* stream);

size_t bb_decode_step_workspace(int64_t cap, int H, int Hkv, int D, int front, int window, int routed);

/*
 * Cache compaction for kv_evict: dst[h, i, :] = src[h, idx[h, i], :] for heads x m rows of D 16-bit elements
 * (D % 8 == 0); src [heads, n_src, D] strides ss[2], dst strides sd[2] (head, row), idx int64 [heads, m] with row
 * stride si0; an index outside [0, n_src) gives a zero row. Replaces the K/V gather of RDAttention.evict
 * (modal_rd/attention.py:253-257).
 */
int bb_gather_rows(const void* src, const int64_t* ss, int64_t n_src, int heads, const int64_t* idx, int64_t si0, int m,
                   int D, void* dst, const int64_t* sd, void* stream);

/*
 * Per row of vals [rows, n] fp32 (row stride sv0): the `budget` columns in [front, n - tail) with the largest
 * values (values <= 0 and NaN rank last; ties to the lower index), ascending int32 in out [rows, budget], -1 past
 * the eligible count. Replaces prio.topk(extra).indices.sort() of RDAttention.evict (modal_rd/attention.py:251-252).
 */
int bb_topk_f32(const float* vals, int64_t sv0, int rows, int64_t n, int front, int tail, int budget, int32_t* out,
                void* ws, size_t ws_bytes, void* stream);
size_t bb_topk_f32_workspace(int rows, int64_t n);

/*
 * Greedy token choice of a decode step: out[0] (int64, device) = index of the largest element of x [n] (dtype 0
 * fp32, 1 bf16, 2 fp16; contiguous); a NaN counts as larger than every number and the first index wins ties
 * (torch.argmax). One workgroup, no workspace: safe inside a captured decode graph. Replaces
 * logits[0, -1].argmax() of StaticDecoder.step (modal_rd/graph_decode.py:201-202).
 */
int bb_argmax(const void* x, int64_t n, int dtype, int64_t* out, void* stream);

/*
 * RMSNorm of `rows` rows of x (row stride sx elements, D contiguous 16-bit values, bf16 or fp16 by is_f16) with
 * weight w [D] into out (row stride so): the arithmetic of transformers' LlamaRMSNorm (fp32 mean of squares,
 * rsqrt(mean + eps), round to the model dtype, times the weight, round). One launch per call, for the decode step's
 * input / post-attention / final norms (modal_rd/graph_decode.py:185,200-201, which run the HF modules).
 */
int bb_rms_norm(const void* x, int64_t sx, int rows, int D, const void* w, float eps, int is_f16, void* out,
                int64_t so, void* stream);

/*
 * A decoder layer's residual add followed by the next RMSNorm, in one launch: sum = round(x + res) (a 16-bit tensor
 * add), out = bb_rms_norm(sum). x, res, sum, out are `rows` rows of D values (row strides sx, sr, ssum, so; sum and
 * out must not overlap x or res). Same limits as bb_rms_norm. Replaces `hidden + attn_out` / `hidden + mlp_out` and
 * the norm after it in the HF decoder layers that the decode step runs (modal_rd/graph_decode.py:185,199-201).
 */
int bb_add_rms_norm(const void* x, int64_t sx, const void* res, int64_t sr, int rows, int D, const void* w, float eps,
                    int is_f16, void* sum, int64_t ssum, void* out, int64_t so, void* stream);

/*
 * out = round(round(silu(g)) u) over n 16-bit values (bf16 or fp16 by is_f16; n % 8 == 0; 16-byte aligned buffers):
 * the arithmetic of F.silu(gate) * up in a Llama MLP (silu in fp32 as g / (1 + exp(-g))), one launch. Replaces
 * `act_fn(gate_proj(x)) * up_proj(x)` of the decode step's MLP (modal_rd/graph_decode.py:200, the HF module).
 */
int bb_silu_mul(const void* g, const void* u, int64_t n, int is_f16, void* out, void* stream);

/*
 * One token through a linear layer: y[N] = W[N, K] x[K] (W row stride sw >= K elements; 16-bit W, x, y, bf16 or
 * fp16 by is_f16; fp32 accumulation, y rounded once). K % 8 == 0, K <= 16384; W rows and x 16-byte aligned. With
 * glu, W holds 2N rows (a Llama MLP's gate rows [0, N) above its up rows [N, 2N)) and y[i] = bb_silu_mul of the
 * rounded gate and up outputs i: the MLP's down-projection input in one launch. Replaces the bias-free projections
 * of the decode step (q/k/v, o, gate / up, down: vendor GEMMs through nn.Linear in
 * modal_rd/graph_decode.py:186-188,199-200); HBM-bound on streaming W once.
 */
int bb_gemv(const void* w, int64_t sw, int N, int K, const void* x, int glu, int is_f16, void* y, void* stream);

/*
 * bb_gemv on the RMSNorm of a hidden row: y = W rms_norm(x + res) with norm weight norm_w [K] and eps, where sum =
 * x + res is also written (res and sum both null: no add). Bit-identical to bb_add_rms_norm (or bb_rms_norm)
 * followed by bb_gemv, in one launch (every workgroup normalises the row itself). K <= 8192; sum must not overlap x
 * or res. Replaces a decoder layer's residual add, norm and following projection in the decode step
 * (modal_rd/graph_decode.py:185-188,199-200).
 */
int bb_gemv_norm(const void* w, int64_t sw, int N, int K, const void* x, const void* res, const void* norm_w,
                 float eps, int glu, int is_f16, void* sum, void* y, void* stream);

/*
 * In-place RoPE on x [B, Hh, T, D] (strides sx[3]) with cos/sin [B, T, D] (strides sc[2]; 0 to broadcast), with
 * the arithmetic of HF apply_rotary_pos_emb on bf16 (is_f16 = 0) or fp16 (is_f16 = 1) tensors (bit-identical).
 * Replaces rope_inplace (modal_rd/attention.py:51-60).
 */
int bb_rope_inplace(void* x, const int64_t* sx, int B, int Hh, int64_t T, int D, const void* cos, const void* sin,
                    const int64_t* sc, int is_f16, void* stream);

/*
 * Measurement helper (no reference counterpart): reads `bytes` (a multiple of 16, 16-byte aligned) of device memory
 * with non-temporal 16-byte loads, one contiguous range per each of `workgroups` workgroups of 256 threads, and
 * writes one XOR word per workgroup to sink[workgroups]. Over a buffer far larger than the 256 MB Infinity Cache its rate is the HBM read ceiling the
 * decode kernels are reported against, next to the published 8 TB/s.
 */
int bb_stream_read(const void* buf, size_t bytes, uint32_t* sink, int workgroups, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BB_ATTN_H */
