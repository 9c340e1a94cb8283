// INT8 KV cache kernels (modal_rd/kv_int8.py:15-26 and kernels/kv_int8_triton.py:14-33 of the reference) and the
// fused exact decode over the int8 cache (modal_rd/attention.py:137-141 run on the dequantised cache there).
//
//   quantize    scale = max(absmax(row) / 127, min_scale) in fp32 (correctly rounded divide), q = rint(x / scale)
//               clamped to [-127, 127]; the scale is stored as fp16 (RNE, the reference's format) or fp32.
//   dequantize  q * float(scale) -> bf16 (RNE) or fp32.
//   decode      one query token per head against n cached rows, K/V read as int8 straight from the token-major
//               cache [cap, Hkv, D] (no dequantised copy): flash-decoding split over keys, each workgroup owns one
//               KV head and a key range and serves all G query heads of that group, so every K/V byte is read once.
#include <hip/hip_fp16.h>

#include "bb_common.h"
#include "bb_internal.h"

namespace bb {
namespace {

BB_DEV float load_scale(const void* s, int64_t i, int is_f16) {
  if (is_f16) return __half2float(reinterpret_cast<const __half*>(s)[i]);
  return reinterpret_cast<const float*>(s)[i];
}

// One group of D/8 lanes per row, 8 elements per lane. blockIdx.y picks one of two (input, int8, scale) sets of the
// same shape: a decode step quantises its new K row and V row in one launch.
struct QuantSet {
  const void* x;
  int8_t* q;
  void* s;
};

// Quantises the 8 elements v of one row whose LPR lanes form an aligned group of the wave (each holds 8 elements of
// the row): scale = max(absmax / 127, min_scale), q = rint(x / scale) clamped to [-127, 127], packed little-endian.
// Every lane of the group must take part (the absmax goes through lane shuffles).
template <int LPR>
BB_DEV float quant8(const float (&v)[8], float min_scale, uint32_t (&packed)[2]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  float scale = amax / 127.0f;
  scale = scale < min_scale ? min_scale : scale;
  packed[0] = packed[1] = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float qv = rintf(v[i] / scale);
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    packed[i >> 2] |= ((uint32_t)(uint8_t)(int8_t)qv) << (8 * (i & 3));
  }
  return scale;
}

BB_DEV void store_scale(void* s, int64_t i, float scale, int is_f16) {
  if (is_f16) reinterpret_cast<__half*>(s)[i] = __float2half_rn(scale);
  else reinterpret_cast<float*>(s)[i] = scale;
}

// Element kinds of the quantise input and the dequantise output (bb_int8_quantize / bb_int8_dequantize).
constexpr int kKindBf16 = 0, kKindF32 = 1, kKindF16 = 2;

template <int D>
__global__ __launch_bounds__(256) void quantize_kernel(QuantSet set0, QuantSet set1, int x_kind, int64_t rows,
                                                       int64_t row_stride, int inner, int64_t inner_stride,
                                                       float min_scale, int scale_is_f16) {
  const QuantSet& set = blockIdx.y ? set1 : set0;
  const void* __restrict__ x = set.x;
  int8_t* __restrict__ qo = set.q;
  void* __restrict__ so = set.s;
  constexpr int LPR = D / 8;
  constexpr int RPB = 256 / LPR;
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;  // flat row = outer * inner + inner_idx
  const int64_t total = rows * inner;
  const bool valid = r < total;
  float v[8];
  if (valid) {
    const int64_t outer = r / inner, in = r % inner;
    const int64_t off = outer * row_stride + in * inner_stride + 8 * lane_in_row;
    if (x_kind == kKindF32) {
      const float* xp = reinterpret_cast<const float*>(x) + off;
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(xp), b = *reinterpret_cast<const f32x4_t*>(xp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
    } else {  // 16-bit elements, exact in fp32
      const u32x4_t a = ld16(reinterpret_cast<const uint16_t*>(x) + off);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t h = (uint16_t)(a[i >> 1] >> (16 * (i & 1)));
        v[i] = x_kind == kKindF16 ? (float)__builtin_bit_cast(_Float16, h) : bf16_to_f32(h);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  uint32_t packed[2];
  const float scale = quant8<LPR>(v, min_scale, packed);
  if (!valid) return;
  *reinterpret_cast<u32x2_t*>(qo + r * D + 8 * lane_in_row) = u32x2_t{packed[0], packed[1]};
  if (lane_in_row == 0) store_scale(so, r, scale, scale_is_f16);
}

template <int D>
__global__ __launch_bounds__(256) void dequantize_kernel(const int8_t* __restrict__ q, const void* __restrict__ s,
                                                         int scale_is_f16, int64_t rows, void* __restrict__ out,
                                                         int out_kind) {
  constexpr int LPR = D / 8;
  constexpr int RPB = 256 / LPR;
  const int lane_in_row = threadIdx.x % LPR;
  const int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  if (r >= rows) return;
  const float sc = load_scale(s, r, scale_is_f16);
  const u32x2_t w = *reinterpret_cast<const u32x2_t*>(q + r * D + 8 * lane_in_row);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xffu) * sc;
  if (out_kind == kKindF32) {
    float* o = reinterpret_cast<float*>(out) + r * D + 8 * lane_in_row;
    *reinterpret_cast<f32x4_t*>(o) = f32x4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4_t*>(o + 4) = f32x4_t{v[4], v[5], v[6], v[7]};
  } else if (out_kind == kKindF16) {  // round to nearest even, as torch's .to(torch.float16)
    uint32_t w2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w2[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i]) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]) << 16);
    st16(reinterpret_cast<uint16_t*>(out) + r * D + 8 * lane_in_row, u32x4_t{w2[0], w2[1], w2[2], w2[3]});
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + r * D + 8 * lane_in_row;
    st16(o, u32x4_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])});
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Decode. Workgroup (split s, KV head g): 4 waves; a wave walks keys 8 at a time, 8 lanes per key row (16 d each).
constexpr int kDecThreads = 256;
constexpr float kDecRescale = 8.0f;

template <int D, int G, bool INT8>
__global__ __launch_bounds__(kDecThreads) void decode_kernel(DecodeParams p) {
  constexpr int LPK = 8;             // lanes per key
  constexpr int DPL = D / LPK;       // d values per lane
  constexpr int KPW = 64 / LPK;      // keys per wave step
  constexpr int SLOTS = kDecThreads / LPK;  // key slots per workgroup (32)
  __shared__ float part_m[SLOTS][G];
  __shared__ float part_l[SLOTS][G];
  __shared__ float part_o[SLOTS][G][D];

  const int split = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kslot = lane / LPK, sub = lane % LPK;
  const int slot = wave * KPW + kslot;
  const int64_t j_begin = (int64_t)split * p.split_len;
  int64_t j_end = j_begin + p.split_len;
  if (j_end > p.n) j_end = p.n;

  float qv[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qr = p.q + (int64_t)(g * G + h) * p.sq + DPL * sub;
#pragma unroll
    for (int e = 0; e < DPL; ++e) qv[h][e] = bf16_to_f32(qr[e]);
  }
  float m[G], l[G], acc[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -1.0e20f;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.0f;
  }

  for (int64_t j = j_begin + slot; j < j_end; j += SLOTS) {
    float kf[DPL], vf[DPL];
    float ks = 1.0f, vs = 1.0f;
    if constexpr (INT8) {
      const int64_t row = j * p.Hkv + g;
      const int8_t* kr = p.k8 + row * D + DPL * sub;
      const int8_t* vr = p.v8 + row * D + DPL * sub;
      ks = load_scale(p.ks, row, p.scale_is_f16);
      vs = load_scale(p.vs, row, p.scale_is_f16);
#pragma unroll
      for (int e0 = 0; e0 < DPL; e0 += 16) {
        const u32x4_t kw = ld16(kr + e0), vw = ld16(vr + e0);
#pragma unroll
        for (int e = 0; e < 16 && e0 + e < DPL; ++e) {
          kf[e0 + e] = (float)(int8_t)((kw[e >> 2] >> (8 * (e & 3))) & 0xffu);
          vf[e0 + e] = (float)(int8_t)((vw[e >> 2] >> (8 * (e & 3))) & 0xffu);
        }
      }
    } else {
      const uint16_t* kr = p.kb + (int64_t)g * p.skb0 + j * p.skb1 + DPL * sub;
      const uint16_t* vr = p.vb + (int64_t)g * p.svb0 + j * p.svb1 + DPL * sub;
#pragma unroll
      for (int e0 = 0; e0 < DPL; e0 += 8) {
        const u32x4_t kw = ld16(kr + e0), vw = ld16(vr + e0);
#pragma unroll
        for (int e = 0; e < 8 && e0 + e < DPL; ++e) {
          kf[e0 + e] = bf16_to_f32((uint16_t)(kw[e >> 1] >> (16 * (e & 1))));
          vf[e0 + e] = bf16_to_f32((uint16_t)(vw[e >> 1] >> (16 * (e & 1))));
        }
      }
    }
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float t = 0.0f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) t = fmaf(qv[h][e], kf[e], t);
      s[h] = t;
    }
#pragma unroll
    for (int off = 1; off < LPK; off <<= 1)
#pragma unroll
      for (int h = 0; h < G; ++h) s[h] += __shfl_xor(s[h], off);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = s[h] * ks * p.c;
      if (x > m[h] + kDecRescale) {
        const float alpha = fast_exp2(m[h] - x);
        m[h] = x;
        l[h] *= alpha;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[h][e] *= alpha;
      }
      const float pr = fast_exp2(x - m[h]);
      l[h] += pr;
      const float pv = pr * vs;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[h][e] = fmaf(pv, vf[e], acc[h][e]);
    }
  }
  // workgroup combine of the SLOTS partial states per head
  if (sub == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) { part_m[slot][h] = m[h]; part_l[slot][h] = l[h]; }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < DPL; ++e) part_o[slot][h][DPL * sub + e] = acc[h][e];
  __syncthreads();
  for (int t = tid; t < G * D; t += kDecThreads) {
    const int h = t / D, d = t % D;
    float M = -1.0e30f;
    for (int s2 = 0; s2 < SLOTS; ++s2) M = fmaxf(M, part_m[s2][h]);
    float L = 0.0f, O = 0.0f;
    for (int s2 = 0; s2 < SLOTS; ++s2) {
      const float w = fast_exp2(part_m[s2][h] - M);
      L += w * part_l[s2][h];
      O += w * part_o[s2][h][d];
    }
    float* dst = p.part + ((int64_t)(g * G + h) * p.n_splits + split) * (D + 2);
    dst[d] = O;
    if (d == 0) { dst[D] = M; dst[D + 1] = L; }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// MFMA decode for the production shape (head_dim 128, four query heads per KV head, int8 cache). Workgroup (split,
// KV head): 4 waves, wave w taking 32-key chunks w, w + 4, ... of the split's key range. Per chunk a wave
//   * streams the chunk's 32 K rows and 32 V rows (int8, 128 bytes each) straight into its own LDS buffers, one
//     chunk ahead, with non-temporal 16-byte buffer loads in which every instruction covers 8 whole rows (rows are
//     read once per step; non-temporal loads stream at about 7.1 TB/s against 6.2 TB/s for plain ones when each
//     instruction covers whole 128-byte lines, and slower than plain ones when it covers parts of lines, as a lane
//     layout of one key per lane would); the buffer resources read rows past n as zeros. Piece c of row r sits in
//     16-byte slot c ^ ((r >> 1) & 7), so the operand reads below are free of bank conflicts;
//   * computes S = Q K^T on one 32x32x16 bf16 MFMA column block (rows 0..3 of Q are the four heads, rows 4..31 are
//     zero; int8 values are exact in bf16). The contraction runs over d in the order 64 hh + 8 dk + e on both
//     operands, so a lane's K operand is one half row, read from LDS;
//   * runs the online softmax on lanes 0..31 (one key each) for the four heads, with the exponent offset moved only
//     when a probability would exceed 2^8, and stores P (times the V row scale) to LDS as bf16 [head][key];
//   * reads the V rows back with ds_read_b64_tr_b8, which hands each lane 8 keys of one d: the V^T operand;
//   * accumulates O^T += V^T P^T on 8 MFMAs (4 blocks of 32 d x 2 steps of 16 keys).
// The four waves' states merge through LDS into one partial (m, l, o) per head and split for decode_merge_kernel.
constexpr int kMdWaves = 4;
constexpr int kMdChunk = 32;    // keys per wave step
constexpr int kMdStages = 2;    // chunk buffers per wave (the next chunk lands while this one is computed)
struct MdLds {
  uint8_t kv[kMdWaves][kMdStages][2][kMdChunk * 128];  // per wave and stage: the K rows, then the V rows
  uint16_t pt[kMdWaves][4 * kMdChunk + 8];  // P^T bf16 [head][key], then one zero 16-byte block
  float m[kMdWaves][4];
  float l[kMdWaves][4];
  float o[kMdWaves][4][128];
};
typedef int v2i_t __attribute__((ext_vector_type(2)));

BB_DEV u32x2_t i8x4_to_bf16x4(uint32_t w) {
  return u32x2_t{pack_bf16x2((float)(int8_t)(w & 0xffu), (float)(int8_t)((w >> 8) & 0xffu)),
                 pack_bf16x2((float)(int8_t)((w >> 16) & 0xffu), (float)(int8_t)(w >> 24))};
}
BB_DEV bf16x8_t i8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
  const u32x2_t a = i8x4_to_bf16x4(w0), b = i8x4_to_bf16x4(w1);
  return as_bf16x8(u32x4_t{a[0], a[1], b[0], b[1]});
}
BB_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
BB_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <bool F16S>
__global__ __launch_bounds__(64 * kMdWaves, 2) void decode_mfma_kernel(DecodeParams p) {
  __shared__ __attribute__((aligned(16))) MdLds sm;
  constexpr int D = 128;
  const int split = blockIdx.x, g = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, hh = lane >> 5;
  const int64_t j_begin = (int64_t)split * p.split_len;
  const int64_t j_end = j_begin + p.split_len < p.n ? j_begin + p.split_len : p.n;

  // The step's new token sits in row n - 1, inside the last split: that split's workgroup quantises its KV head's K
  // and V row into the cache (lanes 0..15 the K row, 16..31 the V row, 8 elements each; quantize_kernel's
  // arithmetic) before any of its waves reads the rows. The workgroup's waves share one L1, so the barrier makes the
  // stores visible to their loads.
  if (p.knew != nullptr && split == p.n_splits - 1) {
    if (wave == 0 && lane < 32) {
      const int part = lane >> 4, lr = lane & 15;
      const uint16_t* src = part ? p.vnew + (int64_t)g * p.svnew : p.knew + (int64_t)g * p.sknew;
      const u32x4_t a = ld16(src + 8 * lr);
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_to_f32((uint16_t)(a[i] & 0xffffu));
        v[2 * i + 1] = bf16_to_f32((uint16_t)(a[i] >> 16));
      }
      uint32_t packed[2];
      const float sc = quant8<16>(v, p.min_scale, packed);
      const int64_t r = (p.n - 1) * p.Hkv + g;
      *reinterpret_cast<u32x2_t*>((part ? p.wv8 : p.wk8) + r * D + 8 * lr) = u32x2_t{packed[0], packed[1]};
      if (lr == 0) store_scale(part ? p.wvs : p.wks, r, sc, p.scale_is_f16);
    }
    __syncthreads();
  }

  bf16x8_t qa[8];  // Q rows 0..3 = query heads 4g..4g+3; fragment dk holds d = 64 hh + 8 dk + 0..7
#pragma unroll
  for (int dk = 0; dk < 8; ++dk)
    qa[dk] = as_bf16x8(li < 4 ? ld16(p.q + (int64_t)(4 * g + li) * p.sq + 64 * hh + 8 * dk) : u32x4_t{0, 0, 0, 0});

  // one buffer resource per cache over KV head g's rows up to this split's end (row j at byte j * row_bytes): the
  // rows a split's last, partial 32-key chunk reaches past it read as 0 instead of being fetched
  const int64_t row_bytes = (int64_t)p.Hkv * D;
  const int range = (int)((j_end - 1) * row_bytes + D);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.k8 + (int64_t)g * D), 0, range, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(p.v8 + (int64_t)g * D), 0, range, 0x00020000);

  float m[4], l[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) { m[h] = -1.0e20f; l[h] = 0.0f; }
  f32x16_t o[4];
#pragma unroll
  for (int dv = 0; dv < 4; ++dv) o[dv] = f32x16_t{};
  uint16_t* pl = sm.pt[wave];
  if (lane < 8) pl[4 * kMdChunk + lane] = 0;  // the zero block read by the lanes of query columns 4..31

  // row r's 16-byte piece c at slot c ^ swz(r) of its 128-byte LDS row
  auto swz = [](int r) { return (r >> 1) & 7; };
  // Chunk c's rows into stage st: direct load i (of 4 per tensor) fills rows 8 i .. 8 i + 7, lane l landing at byte
  // 16 l of that 1 KB: row 8 i + l / 8, slot l % 8, i.e. global piece (l % 8) ^ swz(row). Every instruction reads 8
  // whole 128-byte rows. Returns the chunk's scales (plain loads; the scale rows of the 8 KV heads share lines).
  struct Scales {
    float ks, vs;
  };
  auto fetch = [&](int64_t c, int st, Scales& sc) {
    const int64_t key0 = j_begin + c * kMdChunk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 8 * i + (lane >> 3);
      const uint32_t off = (uint32_t)((key0 + row) * row_bytes) + 16u * (uint32_t)((lane & 7) ^ swz(row));
#pragma unroll
      for (int t = 0; t < 2; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            t ? vrs : krs, reinterpret_cast<__attribute__((address_space(3))) void*>(
                               reinterpret_cast<uintptr_t>(&sm.kv[wave][st][t][1024 * i])),
            16, off, 0, 0, 2 /* non-temporal */);
    }
    const int64_t key = key0 + li;
    const int64_t si = (key < j_end ? key : j_end - 1) * p.Hkv + g;
    if constexpr (F16S) {
      sc.ks = __half2float(reinterpret_cast<const __half*>(p.ks)[si]);
      sc.vs = __half2float(reinterpret_cast<const __half*>(p.vs)[si]);
    } else {
      sc.ks = reinterpret_cast<const float*>(p.ks)[si];
      sc.vs = reinterpret_cast<const float*>(p.vs)[si];
    }
  };
  const int64_t nchunks = (j_end - j_begin + kMdChunk - 1) / kMdChunk;
  Scales cur;
  int st = 0;
  if (wave < nchunks) fetch(wave, 0, cur);
  for (int64_t c = wave; c < nchunks; c += kMdWaves) {
    // unconditional, so the wait count stays exact: past the last chunk this re-reads the current one
    Scales nxt;
    fetch(c + kMdWaves < nchunks ? c + kMdWaves : c, st ^ 1, nxt);
    // this chunk's 8 direct loads have landed once at most the 10 vector-memory operations just issued (8 direct
    // loads and 2 scale loads) are outstanding
    __builtin_amdgcn_s_waitcnt(0x0F7A);  // vmcnt(10)
    const uint8_t* kl = sm.kv[wave][st][0];
    const uint8_t* vl = sm.kv[wave][st][1];
    const int64_t key = j_begin + c * kMdChunk + li;
    const bool valid = hh == 0 && key < j_end;
    u32x4_t kr[4];  // the lane's half row: pieces 4 hh + c4 of row li
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4)
      kr[c4] = *reinterpret_cast<const u32x4_t*>(kl + 128 * li + 16 * ((4 * hh + c4) ^ swz(li)));
    const float ksc = cur.ks, vsc = cur.vs;
    // S = Q K^T: lane (key li, hh = 0) gets the four heads' scores in elements 0..3
    f32x16_t sacc = f32x16_t{};
#pragma unroll
    for (int dk = 0; dk < 8; ++dk)
      sacc = mfma32(qa[dk], i8x8_to_bf16x8(kr[dk >> 1][2 * (dk & 1)], kr[dk >> 1][2 * (dk & 1) + 1]), sacc);
    float x[4], pr[4];
    bool over = false;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      x[h] = valid ? sacc[h] * ksc * p.c : -__builtin_huge_valf();
      pr[h] = fast_exp2(x[h] - m[h]);
      over |= !(pr[h] <= 256.0f);
    }
    if (__builtin_amdgcn_ballot_w64(over)) {
      float alpha_lane = 1.0f;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float mn = fmaxf(m[h], wave_max(x[h]));
        const float alpha = fast_exp2(m[h] - mn);
        m[h] = mn;
        l[h] *= alpha;
        if (li == h) alpha_lane = alpha;
        pr[h] = fast_exp2(x[h] - m[h]);
      }
#pragma unroll
      for (int dv = 0; dv < 4; ++dv)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dv][r] *= alpha_lane;
    }
    // P^T (times the V row scale) to LDS
    if (hh == 0) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        l[h] += pr[h];
        pl[h * kMdChunk + li] = f32_to_bf16(pr[h] * vsc);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O^T += V^T P^T
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8_t pb = as_bf16x8(ld16(li < 4 ? pl + li * kMdChunk + 16 * ks + 8 * hh : pl + 4 * kMdChunk));
      const int s16 = lane & 15;
      const int src_key = 16 * ks + 8 * hh + (s16 >> 1);
#pragma unroll
      for (int dv = 0; dv < 4; ++dv) {
        const int src_d = 32 * dv + 16 * ((lane >> 4) & 1) + 8 * (s16 & 1);
        const v2i_t t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            reinterpret_cast<__attribute__((address_space(3))) v2i_t*>(reinterpret_cast<uintptr_t>(
                vl + 128 * src_key + 16 * ((src_d >> 4) ^ swz(src_key)) + (src_d & 15))));
        o[dv] = mfma32(i8x8_to_bf16x8((uint32_t)t.x, (uint32_t)t.y), pb, o[dv]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    cur = nxt;
    st ^= 1;
  }
  // the loop's last fetch (a repeat of its last chunk) must land before the workgroup's LDS is reused or released
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // merge the four waves: m is wave-uniform, l is spread over the key lanes, O^T column h sits in lanes h and h + 32
#pragma unroll
  for (int h = 0; h < 4; ++h) l[h] = wave_sum(l[h]);
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < 4; ++h) { sm.m[wave][h] = m[h]; sm.l[wave][h] = l[h]; }
  }
  if (li < 4) {
#pragma unroll
    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
      for (int r = 0; r < 16; ++r) sm.o[wave][li][32 * dv + 8 * (r >> 2) + 4 * hh + (r & 3)] = o[dv][r];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < 4 * D; t += 64 * kMdWaves) {
    const int h = t / D, d = t % D;
    float M = sm.m[0][h];
#pragma unroll
    for (int w = 1; w < kMdWaves; ++w) M = fmaxf(M, sm.m[w][h]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kMdWaves; ++w) {
      const float wt = fast_exp2(sm.m[w][h] - M);
      L += wt * sm.l[w][h];
      O += wt * sm.o[w][h][d];
    }
    float* dst = p.part + ((int64_t)(4 * g + h) * p.n_splits + split) * (D + 2);
    dst[d] = O;
    if (d == 0) { dst[D] = M; dst[D + 1] = L; }
  }
}

// the MFMA decode addresses KV head g's rows with 32-bit buffer offsets, including the rows of a last partial chunk
bool decode_mfma_fits(const DecodeParams& p) {
  return (p.n + kMdChunk) * (int64_t)p.Hkv * 128 < ((int64_t)1 << 31);
}

// Split merge: a workgroup per (query head, 16 columns), so that the partials are read by 8x as many CUs. Thread
// (column, group) folds every 16th split of its column with a running maximum, loading 8 splits at a time; the 16
// groups then combine through LDS.
constexpr int kMergeThreads = 256;
constexpr int kMergeCols = 16;
constexpr int kMergeGroups = kMergeThreads / kMergeCols;
constexpr int kMergePer = 8;
template <int D>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(DecodeParams p) {
  __shared__ float sm_m[kMergeGroups], sm_l[kMergeGroups], sm_o[kMergeGroups][kMergeCols];
  const int h = blockIdx.x, t = threadIdx.x, dl = t % kMergeCols, grp = t / kMergeCols;
  const int d = kMergeCols * blockIdx.y + dl;
  const int ns = p.n_splits;
  const float* base = p.part + (int64_t)h * ns * (D + 2);
  float M = -1.0e30f, L = 0.0f, O = 0.0f;
  for (int i0 = 0; grp + kMergeGroups * i0 < ns; i0 += kMergePer) {
    float mv[kMergePer], lv[kMergePer], ov[kMergePer];
#pragma unroll
    for (int i = 0; i < kMergePer; ++i) {
      const int s = grp + kMergeGroups * (i0 + i);
      const bool ok = s < ns;
      const float* r = base + (int64_t)(ok ? s : 0) * (D + 2);
      mv[i] = ok ? r[D] : -1.0e30f;
      lv[i] = ok ? r[D + 1] : 0.0f;
      ov[i] = ok ? r[d] : 0.0f;
    }
    float mn = M;
#pragma unroll
    for (int i = 0; i < kMergePer; ++i) mn = fmaxf(mn, mv[i]);
    const float a = fast_exp2(M - mn);
    L *= a;
    O *= a;
#pragma unroll
    for (int i = 0; i < kMergePer; ++i) {
      const float w = fast_exp2(mv[i] - mn);
      L += w * lv[i];
      O += w * ov[i];
    }
    M = mn;
  }
  sm_o[grp][dl] = O;
  if (dl == 0) { sm_m[grp] = M; sm_l[grp] = L; }
  __syncthreads();
  if (grp == 0) {
    float mx = sm_m[0];
#pragma unroll
    for (int g2 = 1; g2 < kMergeGroups; ++g2) mx = fmaxf(mx, sm_m[g2]);
    float lt = 0.0f, ot = 0.0f;
#pragma unroll
    for (int g2 = 0; g2 < kMergeGroups; ++g2) {
      const float w = fast_exp2(sm_m[g2] - mx);
      lt += w * sm_l[g2];
      ot += w * sm_o[g2][dl];
    }
    p.out[(int64_t)h * p.so + d] = f32_to_bf16(ot / fmaxf(lt, 1.0e-20f));
  }
}

template <int D, int G>
hipError_t launch_decode_dg(const DecodeParams& p, hipStream_t stream) {
  if (D == 128 && G == 4 && p.k8 && decode_mfma_fits(p)) {
    if (p.scale_is_f16)
      hipLaunchKernelGGL(decode_mfma_kernel<true>, dim3(p.n_splits, p.Hkv), dim3(64 * kMdWaves), 0, stream, p);
    else
      hipLaunchKernelGGL(decode_mfma_kernel<false>, dim3(p.n_splits, p.Hkv), dim3(64 * kMdWaves), 0, stream, p);
  } else if (p.k8)
    hipLaunchKernelGGL((decode_kernel<D, G, true>), dim3(p.n_splits, p.Hkv), dim3(kDecThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_kernel<D, G, false>), dim3(p.n_splits, p.Hkv), dim3(kDecThreads), 0, stream, p);
  hipLaunchKernelGGL(decode_merge_kernel<D>, dim3(p.H, D / kMergeCols), dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

template <int D>
hipError_t launch_decode_d(const DecodeParams& p, hipStream_t stream) {
  switch (p.H / p.Hkv) {
    case 1: return launch_decode_dg<D, 1>(p, stream);
    case 2: return launch_decode_dg<D, 2>(p, stream);
    case 4: return launch_decode_dg<D, 4>(p, stream);
    case 8: return launch_decode_dg<D, 8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// RoPE: x' = r(r(x * cos) + r(rotate_half(x) * sin)), rotate_half(x) = cat(-x2, x1), r = rounding to the tensor
// dtype (bf16, or fp16 when F16): the arithmetic of HF apply_rotary_pos_emb on 16-bit tensors (each torch op computes
// in fp32 and rounds to the tensor dtype), so results are bit-identical.
template <bool F16>
BB_DEV float from16(uint16_t h) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, h);
  else return bf16_to_f32(h);
}

// x rounded to the element type and back, as one materialised value. HF rounds each product before the add; for fp16
// the compiler would otherwise shrink the rounding into a half-precision multiply and fuse it with the add (one fma,
// one rounding), so the rounded bits pass through an empty asm it cannot see into.
template <bool F16>
BB_DEV float round16(float x) {
  uint32_t h = to16<F16>(x);
  asm volatile("" : "+v"(h));
  return from16<F16>((uint16_t)h);
}

template <bool F16>
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* __restrict__ x, int64_t sx0, int64_t sx1, int64_t sx2,
                                                   int B, int Hh, int64_t T, int D, const uint16_t* __restrict__ cs,
                                                   const uint16_t* __restrict__ sn, int64_t sc0, int64_t sc1) {
  const int half = D / 2;
  const int cpr = half / 8;  // 8-element chunks per half row
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * Hh * T * cpr;
  if (t >= total) return;
  // head fastest: the Hh rows of one position share their cos / sin row, which then stays in cache (with the
  // position fastest every head would stream the whole cos / sin table again)
  const int c = (int)(t % cpr);
  const int64_t row = t / cpr;
  const int64_t hh = row % Hh;
  const int64_t bp = row / Hh;
  const int64_t pos = bp % T, b = bp / T;
  uint16_t* xr = x + b * sx0 + hh * sx1 + pos * sx2;
  const uint16_t* cr = cs + b * sc0 + pos * sc1;
  const uint16_t* sr = sn + b * sc0 + pos * sc1;
  const int d1 = 8 * c, d2 = half + 8 * c;
  const u32x4_t x1 = ld16(xr + d1), x2 = ld16(xr + d2);
  const u32x4_t c1 = ld16(cr + d1), c2 = ld16(cr + d2);
  const u32x4_t s1 = ld16(sr + d1), s2 = ld16(sr + d2);
  u32x4_t o1, o2;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t r1 = 0, r2 = 0;
#pragma unroll
    for (int hw = 0; hw < 2; ++hw) {
      const int sh = 16 * hw;
      const float a1 = from16<F16>((uint16_t)(x1[w] >> sh)), a2 = from16<F16>((uint16_t)(x2[w] >> sh));
      const float fc1 = from16<F16>((uint16_t)(c1[w] >> sh)), fc2 = from16<F16>((uint16_t)(c2[w] >> sh));
      const float fs1 = from16<F16>((uint16_t)(s1[w] >> sh)), fs2 = from16<F16>((uint16_t)(s2[w] >> sh));
      // first half: x1*cos1 + (-x2)*sin1 ; second half: x2*cos2 + x1*sin2
      const float p1 = round16<F16>(a1 * fc1);
      const float q1 = round16<F16>(-a2 * fs1);
      const float p2 = round16<F16>(a2 * fc2);
      const float q2 = round16<F16>(a1 * fs2);
      r1 |= (uint32_t)to16<F16>(p1 + q1) << sh;
      r2 |= (uint32_t)to16<F16>(p2 + q2) << sh;
    }
    o1[w] = r1;
    o2[w] = r2;
  }
  st16(xr + d1, o1);
  st16(xr + d2, o2);
}

}  // namespace

hipError_t launch_int8_quantize(const void* x, int x_kind, int64_t rows, int64_t row_stride, int inner,
                                int64_t inner_stride, int D, float min_scale, int8_t* q, void* scale, int scale_is_f16,
                                hipStream_t stream, const void* x1, int8_t* q1, void* scale1) {
  const int64_t total = rows * inner;
  if (total <= 0) return hipSuccess;
  const int rpb = 256 / (D / 8);
  const dim3 grid((unsigned)((total + rpb - 1) / rpb), x1 ? 2u : 1u);
  const QuantSet s0{x, q, scale}, s1{x1 ? x1 : x, x1 ? q1 : q, x1 ? scale1 : scale};
  switch (D) {
    case 32: hipLaunchKernelGGL(quantize_kernel<32>, grid, dim3(256), 0, stream, s0, s1, x_kind, rows, row_stride, inner, inner_stride, min_scale, scale_is_f16); break;
    case 64: hipLaunchKernelGGL(quantize_kernel<64>, grid, dim3(256), 0, stream, s0, s1, x_kind, rows, row_stride, inner, inner_stride, min_scale, scale_is_f16); break;
    case 128: hipLaunchKernelGGL(quantize_kernel<128>, grid, dim3(256), 0, stream, s0, s1, x_kind, rows, row_stride, inner, inner_stride, min_scale, scale_is_f16); break;
    case 256: hipLaunchKernelGGL(quantize_kernel<256>, grid, dim3(256), 0, stream, s0, s1, x_kind, rows, row_stride, inner, inner_stride, min_scale, scale_is_f16); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_int8_dequantize(const int8_t* q, const void* scale, int scale_is_f16, int64_t rows, int D, void* out,
                                  int out_kind, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int rpb = 256 / (D / 8);
  const unsigned blocks = (unsigned)((rows + rpb - 1) / rpb);
  switch (D) {
    case 32: hipLaunchKernelGGL(dequantize_kernel<32>, dim3(blocks), dim3(256), 0, stream, q, scale, scale_is_f16, rows, out, out_kind); break;
    case 64: hipLaunchKernelGGL(dequantize_kernel<64>, dim3(blocks), dim3(256), 0, stream, q, scale, scale_is_f16, rows, out, out_kind); break;
    case 128: hipLaunchKernelGGL(dequantize_kernel<128>, dim3(blocks), dim3(256), 0, stream, q, scale, scale_is_f16, rows, out, out_kind); break;
    case 256: hipLaunchKernelGGL(dequantize_kernel<256>, dim3(blocks), dim3(256), 0, stream, q, scale, scale_is_f16, rows, out, out_kind); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

size_t decode_workspace_bytes(int H, int D, int n_splits) { return (size_t)H * n_splits * (D + 2) * sizeof(float); }

bool decode_fuses_append(const DecodeParams& p) {
  return p.D == 128 && p.H == 4 * p.Hkv && p.k8 != nullptr && decode_mfma_fits(p);
}

hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
  if (p.n <= 0) return hipErrorInvalidValue;
  if (p.knew != nullptr && !decode_fuses_append(p)) return hipErrorInvalidValue;
  switch (p.D) {
    case 64: return launch_decode_d<64>(p, stream);
    case 128: return launch_decode_d<128>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rope(uint16_t* x, int64_t sx0, int64_t sx1, int64_t sx2, int B, int Hh, int64_t T, int D,
                       const uint16_t* cos, const uint16_t* sin, int64_t sc0, int64_t sc1, int f16, hipStream_t stream) {
  const int64_t total = (int64_t)B * Hh * T * (D / 16);
  if (total <= 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (f16)
    hipLaunchKernelGGL(rope_kernel<true>, grid, dim3(256), 0, stream, x, sx0, sx1, sx2, B, Hh, T, D, cos, sin, sc0, sc1);
  else
    hipLaunchKernelGGL(rope_kernel<false>, grid, dim3(256), 0, stream, x, sx0, sx1, sx2, B, Hh, T, D, cos, sin, sc0, sc1);
  return hipGetLastError();
}

}  // namespace bb
