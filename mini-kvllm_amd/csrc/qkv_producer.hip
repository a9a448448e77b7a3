// K6: the producer side of the KV cache, fused: q/k RMSNorm + rotary
// embedding + KV append in one pass over the qkv projection's output.
//
// Reference: Qwen3Attention.forward (qwen3.py:73-118) splits the qkv
// projection into q, k, v, applies q_norm / k_norm (LayerNorm.rms_forward,
// layernorm.py:16-24: x / sqrt(mean(x^2) + eps) * weight) and the rotary
// embedding (rotary_embedding.py:100-109, apply_rotary_pos_emb :4-26: NeoX
// halves, cos / sin from cos_sin_cache[position]), then Attention.forward
// copies k and v to contiguous tensors and appends them
// (attention.py:1654-1691: store_kvcache / store_kvcache_fp8 /
// store_kvcache_int8).  That is six or more launches that each read and
// write the rows again.  Here the rows are read once and the kernel writes q
// (normed, rotated), the rows' K and V in the cache's format (copy, FP8 per
// tensor, FP8 or INT8 per token and head) and, optionally, the rotated k for
// a full-prefill attention over fresh K/V.
//
// Lane layout: a head of D elements is D/16 lanes; lane m of a head holds
// elements [8m, 8m+8) and [D/2 + 8m, D/2 + 8m + 8), i.e. 8 rotary pairs, so
// the rotation is lane-local and only the norm's sum of squares is reduced
// across the head's lanes.
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kProdWaves = 4;

enum ProducerCache { kCacheCopy = 0, kCacheFp8Tensor = 1, kCacheFp8Token = 2, kCacheI8Token = 3 };

struct ProducerArgs {
  const char* qkv;
  int64_t qkv_stride;  // elements per token row of qkv
  int64_t num_tokens;
  int num_heads, num_kv_heads, head_dim;
  const void* q_w;  // q_norm weight (head_dim) or null: no norm
  const void* k_w;
  int w_dtype;
  float eps;
  const void* cos_sin;  // (max_position, head_dim): cos | sin
  int cs_dtype;
  int64_t max_position;
  const int64_t* positions;
  void* q_out;  // (T, num_heads, head_dim), out_dtype
  void* k_out;  // (T, num_kv_heads, head_dim), out_dtype, or null
  int out_dtype;
  char* k_cache;
  char* v_cache;
  int cache_dtype;  // copy mode: the dtype the cache holds
  float* k_scale;
  float* v_scale;
  int calibrate;
  const int64_t* slot_mapping;
  int64_t num_slots;
};

// 8 consecutive elements of dtype dt as fp32.
MKV_DEV void load8_f32(const void* p, int dt, float (&x)[8]) {
  if (dt == MKV_DTYPE_F32) {
    const u32x4 a = ld16(p), b = ld16(reinterpret_cast<const float*>(p) + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = __uint_as_float(a[j]);
      x[4 + j] = __uint_as_float(b[j]);
    }
  } else {
    const u32x4 a = ld16(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool bf = dt == MKV_DTYPE_BF16;
      x[2 * j] = bf ? bf16_bits_to_f32(a[j] & 0xffffu) : f16_bits_to_f32(a[j] & 0xffffu);
      x[2 * j + 1] = bf ? bf16_bits_to_f32(a[j] >> 16) : f16_bits_to_f32(a[j] >> 16);
    }
  }
}

// 8 fp32 values stored as dtype dt (round to nearest even for 16-bit types).
MKV_DEV void store8(void* p, int dt, const float (&x)[8]) {
  if (dt == MKV_DTYPE_F32) {
    st16(p, u32x4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])});
    st16(reinterpret_cast<float*>(p) + 4,
         u32x4{__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7])});
  } else {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool bf = dt == MKV_DTYPE_BF16;
      const uint32_t lo = bf ? f32_to_bf16_bits(x[2 * j]) : f32_to_f16_bits(x[2 * j]);
      const uint32_t hi = bf ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
      w[j] = lo | (hi << 16);
    }
    st16(p, w);
  }
}

MKV_DEV int dtype_bytes(int dt) { return dt == MKV_DTYPE_F32 ? 4 : (dt == MKV_DTYPE_FP8E4M3 || dt == MKV_DTYPE_I8 ? 1 : 2); }

// Sum over the `lanes` lanes of a head (aligned groups of a power of two).
MKV_DEV float head_sum(float v, int lanes) {
  for (int off = 1; off < lanes; off <<= 1) v += __shfl_xor(v, off);
  return v;
}
MKV_DEV float head_max(float v, int lanes) {
  for (int off = 1; off < lanes; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// The lane's 8 + 8 elements of q/k head `head` (element offset of the head in
// the qkv row), normed (if a weight is given) and rotated, in fp32 after
// rounding to out_dtype: the value of the reference's rotated tensor.
//   norm:   y = round_in(x / sqrt(sum(x^2) / D + eps) * w)
//   rotary: o1 = y1 * cos - y2 * sin, o2 = y1 * sin + y2 * cos  (no FMA)
MKV_DEV void produce_qk(const ProducerArgs& a, const char* row, int64_t head_off, const void* w,
                        const float (&wl)[8], const float (&wh)[8], const float (&c)[8],
                        const float (&s)[8], int m, int in_dt, float (&o1)[8], float (&o2)[8]) {
  const int half = a.head_dim / 2;
  const int eb = dtype_bytes(in_dt);
  float x1[8], x2[8];
  load8_f32(row + (head_off + 8 * m) * eb, in_dt, x1);
  load8_f32(row + (head_off + half + 8 * m) * eb, in_dt, x2);
  if (w) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __fadd_rn(ss, __fadd_rn(__fmul_rn(x1[j], x1[j]), __fmul_rn(x2[j], x2[j])));
    ss = head_sum(ss, a.head_dim / 16);
    const float var = __fadd_rn(ss / (float)a.head_dim, a.eps);
    const float r = sqrtf(var);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x1[j] = round_to_dtype(__fmul_rn(x1[j] / r, wl[j]), in_dt);
      x2[j] = round_to_dtype(__fmul_rn(x2[j] / r, wh[j]), in_dt);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    o1[j] = round_to_dtype(__fsub_rn(__fmul_rn(x1[j], c[j]), __fmul_rn(x2[j], s[j])), a.out_dtype);
    o2[j] = round_to_dtype(__fadd_rn(__fmul_rn(x1[j], s[j]), __fmul_rn(x2[j], c[j])), a.out_dtype);
  }
}

// Write the lane's 8 + 8 elements of KV head kvh of slot `slot` into a cache
// row (element offsets 8m and D/2 + 8m of the head).
template <int MODE>
MKV_DEV void store_kv(const ProducerArgs& a, char* cache, float* scales, int64_t slot, int kvh, int m,
                      const float (&o1)[8], const float (&o2)[8], float tensor_scale) {
  const int D = a.head_dim, half = D / 2;
  const int64_t row_elems = (int64_t)a.num_kv_heads * D;
  const int64_t e1 = (int64_t)kvh * D + 8 * m, e2 = e1 + half;
  if constexpr (MODE == kCacheCopy) {
    const int eb = dtype_bytes(a.cache_dtype);
    char* base = cache + slot * row_elems * eb;
    store8(base + e1 * eb, a.cache_dtype, o1);
    store8(base + e2 * eb, a.cache_dtype, o2);
  } else {
    char* base = cache + slot * row_elems;
    float sc = tensor_scale;
    if constexpr (MODE != kCacheFp8Tensor) {
      float am = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) am = fmaxf(am, fmaxf(fabsf(o1[j]), fabsf(o2[j])));
      am = head_max(am, D / 16);
      sc = MODE == kCacheI8Token ? i8_head_scale(am) : fp8_head_scale(am);
      if (m == 0) scales[slot * a.num_kv_heads + kvh] = sc;
    }
    u32x2 w1, w2;
    if constexpr (MODE == kCacheI8Token) {
      const float inv = 1.0f / sc;
      w1 = u32x2{quantize4_i8(o1, inv), quantize4_i8(o1 + 4, inv)};
      w2 = u32x2{quantize4_i8(o2, inv), quantize4_i8(o2 + 4, inv)};
    } else {
      const Fp8Quant q = fp8_quant(sc);
      w1 = u32x2{quantize4_fp8(o1, q), quantize4_fp8(o1 + 4, q)};
      w2 = u32x2{quantize4_fp8(o2, q), quantize4_fp8(o2 + 4, q)};
    }
    *reinterpret_cast<u32x2*>(base + e1) = w1;
    *reinterpret_cast<u32x2*>(base + e2) = w2;
  }
}

// The lane's 8 + 8 elements of V head kvh, as they are: the reference
// appends v as the view of the qkv projection, in the input dtype.
MKV_DEV void load_v(const ProducerArgs& a, const char* row, int kvh, int m, int in_dt, float (&o1)[8],
                    float (&o2)[8]) {
  const int eb = dtype_bytes(in_dt);
  const int64_t off = (int64_t)(a.num_heads + a.num_kv_heads + kvh) * a.head_dim;
  load8_f32(row + (off + 8 * m) * eb, in_dt, o1);
  load8_f32(row + (off + a.head_dim / 2 + 8 * m) * eb, in_dt, o2);
}

// cos / sin of the lane's 8 rotary pairs at `pos`; NaN for a position
// outside the table (no out-of-range read; the outputs become NaN).
MKV_DEV void rotary_row(const ProducerArgs& a, int64_t pos, int m, float (&c)[8], float (&s)[8]) {
  if (pos < 0 || pos >= a.max_position) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = s[j] = __builtin_nanf("");
    return;
  }
  const int eb = dtype_bytes(a.cs_dtype);
  const char* row = reinterpret_cast<const char*>(a.cos_sin) + pos * a.head_dim * eb;
  load8_f32(row + (8 * m) * eb, a.cs_dtype, c);
  load8_f32(row + (a.head_dim / 2 + 8 * m) * eb, a.cs_dtype, s);
}

// Per-tensor FP8 scale still holding the 1.0 sentinel: every wave that sees
// it computes the calibrated scale of the whole call (amax over all rows of
// the rotated k, or of v, slot -1 rows included; NaN wins as in torch.amax),
// exactly as store_kvcache_fp8 calibrates from the key / value it is given,
// and writes it back.  Slow (every wave reads every row); see mkv_kv_append.
MKV_DEV float producer_calibrate(const ProducerArgs& a, bool is_k, float* scale, int in_dt,
                                 const float (&wkl)[8], const float (&wkh)[8]) {
  const int lane = threadIdx.x & (kWave - 1);
  const int lanes = a.head_dim / 16, hpi = kWave / lanes;
  const int m = lane % lanes, hi = lane / lanes;
  uint32_t mx = 0;
  for (int64_t t = 0; t < a.num_tokens; ++t) {
    const char* row = a.qkv + t * a.qkv_stride * dtype_bytes(in_dt);
    float c[8], s[8];
    if (is_k) rotary_row(a, a.positions[t], m, c, s);
    for (int hb = 0; hb < a.num_kv_heads; hb += hpi) {
      const int kvh = hb + hi < a.num_kv_heads ? hb + hi : a.num_kv_heads - 1;
      float o1[8], o2[8];
      if (is_k)
        produce_qk(a, row, (int64_t)(a.num_heads + kvh) * a.head_dim, a.k_w, wkl, wkh, c, s, m, in_dt, o1, o2);
      else
        load_v(a, row, kvh, m, in_dt, o1, o2);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mx = max(mx, __float_as_uint(fabsf(o1[j])));
        mx = max(mx, __float_as_uint(fabsf(o2[j])));
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  // evaluated in the dtype of the tensor the reference calibrates from: the
  // rotated k (out_dtype) or v (the input dtype)
  const int dt = is_k ? a.out_dtype : in_dt;
  const float lo = round_to_dtype(1e-8f, dt);
  float am = __uint_as_float(mx);
  am = am < lo ? lo : am;
  const float sc = round_to_dtype(am / kFp8Max, dt);
  if (lane == 0) *scale = sc;
  return sc;
}

// Work item = (token row, group of heads): the q heads, the k heads and the
// v heads of a row are cut into groups of 64 / (D/16) heads (8 at D = 128),
// one wavefront each, so a row's groups run in parallel and every wave does
// one round of loads, math and stores.
MKV_DEV int head_groups(int heads, int hpi) { return (heads + hpi - 1) / hpi; }

template <int IN_DT, int MODE>
__global__ __launch_bounds__(kProdWaves* kWave) void qkv_producer_kernel(ProducerArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int lanes = a.head_dim / 16, hpi = kWave / lanes;
  const int m = lane % lanes, hi = lane / lanes;
  const int half = a.head_dim / 2;
  const int gq = head_groups(a.num_heads, hpi), gk = head_groups(a.num_kv_heads, hpi);
  const int groups = gq + 2 * gk;
  const int64_t w = (int64_t)blockIdx.x * kProdWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = w / groups;
  if (t >= a.num_tokens) return;
  const int g = (int)(w - t * groups);
  // region of this wave: 0 = q heads, 1 = k heads, 2 = v heads
  const int region = g < gq ? 0 : (g < gq + gk ? 1 : 2);
  const int h = (region == 0 ? g : (region == 1 ? g - gq : g - gq - gk)) * hpi + hi;
  const int region_heads = region == 0 ? a.num_heads : a.num_kv_heads;

  float ks = 0.0f, vs = 0.0f;
  if (MODE == kCacheFp8Tensor && a.slot_mapping && region != 0) {
    // the scale's 1.0 sentinel is handled before the slot test: padding rows
    // count for the calibration
    float wkl[8], wkh[8];
    if (region == 1 && a.k_w) {
      const int eb = dtype_bytes(a.w_dtype);
      load8_f32(reinterpret_cast<const char*>(a.k_w) + (8 * m) * eb, a.w_dtype, wkl);
      load8_f32(reinterpret_cast<const char*>(a.k_w) + (half + 8 * m) * eb, a.w_dtype, wkh);
    }
    if (region == 1) {
      ks = *a.k_scale;
      if (a.calibrate && ks == 1.0f) ks = producer_calibrate(a, true, a.k_scale, IN_DT, wkl, wkh);
    } else {
      vs = *a.v_scale;
      if (a.calibrate && vs == 1.0f) vs = producer_calibrate(a, false, a.v_scale, IN_DT, wkl, wkh);
    }
  }
  if (h >= region_heads) return;  // the last group of a region may be partial
  const char* row = a.qkv + t * a.qkv_stride * DTypeInfo<IN_DT>::kBytes;
  const int ob = dtype_bytes(a.out_dtype);
  const int64_t slot = a.slot_mapping ? a.slot_mapping[t] : -1;
  const bool append = slot >= 0 && slot < a.num_slots;

  if (region == 2) {
    if (!append) return;
    float o1[8], o2[8];
    load_v(a, row, h, m, IN_DT, o1, o2);
    store_kv<MODE>(a, a.v_cache, a.v_scale, slot, h, m, o1, o2, vs);
    return;
  }
  // q or k: norm weights of the lane's elements, cos / sin of the position
  const void* wptr = region == 0 ? a.q_w : a.k_w;
  float wl[8], wh[8];
  if (wptr) {
    const int eb = dtype_bytes(a.w_dtype);
    load8_f32(reinterpret_cast<const char*>(wptr) + (8 * m) * eb, a.w_dtype, wl);
    load8_f32(reinterpret_cast<const char*>(wptr) + (half + 8 * m) * eb, a.w_dtype, wh);
  }
  float c[8], s[8];
  rotary_row(a, a.positions[t], m, c, s);
  float o1[8], o2[8];
  const int64_t head_off = (int64_t)(region == 0 ? h : a.num_heads + h) * a.head_dim;
  produce_qk(a, row, head_off, wptr, wl, wh, c, s, m, IN_DT, o1, o2);
  if (region == 0) {
    char* q = reinterpret_cast<char*>(a.q_out) + ((t * a.num_heads + h) * a.head_dim) * ob;
    store8(q + (8 * m) * ob, a.out_dtype, o1);
    store8(q + (half + 8 * m) * ob, a.out_dtype, o2);
    return;
  }
  if (a.k_out) {
    char* k = reinterpret_cast<char*>(a.k_out) + ((t * a.num_kv_heads + h) * a.head_dim) * ob;
    store8(k + (8 * m) * ob, a.out_dtype, o1);
    store8(k + (half + 8 * m) * ob, a.out_dtype, o2);
  }
  if (append) store_kv<MODE>(a, a.k_cache, a.k_scale, slot, h, m, o1, o2, ks);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_qkv_norm_rope_append(
    const void* qkv, int64_t qkv_row_stride, int in_dtype, int64_t num_tokens, int num_heads,
    int num_kv_heads, int head_dim, const void* q_norm_weight, const void* k_norm_weight,
    int norm_weight_dtype, float eps, const void* cos_sin_cache, int cos_sin_dtype,
    int64_t max_position, const int64_t* positions, void* q_out, void* k_out, int out_dtype,
    void* k_cache, void* v_cache, int cache_dtype, int kv_scale_mode, float* k_scale,
    float* v_scale, const int64_t* slot_mapping, int block_size, int64_t num_blocks, int flags,
    void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || num_blocks < 0 ||
      max_position <= 0)
    return MKV_ERR_BAD_SHAPE;
  if (head_dim < 32 || head_dim > 1024 || (head_dim & (head_dim - 1))) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  if (num_tokens == 0) return MKV_OK;
  if (!qkv || !cos_sin_cache || !positions || !q_out) return MKV_ERR_NULL_POINTER;
  if (slot_mapping && (!k_cache || !v_cache)) return MKV_ERR_NULL_POINTER;
  auto is_float = [](int d) { return d == MKV_DTYPE_F32 || d == MKV_DTYPE_BF16 || d == MKV_DTYPE_F16; };
  if (!is_float(in_dtype) || !is_float(out_dtype) || !is_float(cos_sin_dtype) ||
      ((q_norm_weight || k_norm_weight) && !is_float(norm_weight_dtype)))
    return MKV_ERR_UNSUPPORTED_DTYPE;
  int mode;
  if (is_float(cache_dtype)) {
    mode = kCacheCopy;
  } else if (cache_dtype == MKV_DTYPE_FP8E4M3 && kv_scale_mode == MKV_SCALE_PER_TENSOR) {
    mode = kCacheFp8Tensor;
  } else if (cache_dtype == MKV_DTYPE_FP8E4M3 && kv_scale_mode == MKV_SCALE_PER_TOKEN_HEAD) {
    mode = kCacheFp8Token;
  } else if (cache_dtype == MKV_DTYPE_I8 && kv_scale_mode == MKV_SCALE_PER_TOKEN_HEAD) {
    mode = kCacheI8Token;
  } else {
    return MKV_ERR_UNSUPPORTED_DTYPE;
  }
  if (slot_mapping && mode != kCacheCopy && (!k_scale || !v_scale)) return MKV_ERR_NULL_POINTER;
  if (flags & ~MKV_APPEND_CALIBRATE_SENTINEL) return MKV_ERR_BAD_SHAPE;
  if (qkv_row_stride < (int64_t)(num_heads + 2 * num_kv_heads) * head_dim) return MKV_ERR_BAD_STRIDE;
  const int ib = in_dtype == MKV_DTYPE_F32 ? 4 : 2;
  const int cb = cos_sin_dtype == MKV_DTYPE_F32 ? 4 : 2;
  const int wb = norm_weight_dtype == MKV_DTYPE_F32 ? 4 : 2;
  if (!aligned16(qkv) || (qkv_row_stride * ib) % 16 || !aligned16(cos_sin_cache) || !aligned16(q_out) ||
      (k_out && !aligned16(k_out)) || !aligned16(k_cache) || !aligned16(v_cache) ||
      (q_norm_weight && !aligned16(q_norm_weight)) || (k_norm_weight && !aligned16(k_norm_weight)) ||
      (head_dim * cb) % 16 || (head_dim / 2 * wb) % 16)
    return MKV_ERR_MISALIGNED;

  ProducerArgs a;
  a.qkv = reinterpret_cast<const char*>(qkv);
  a.qkv_stride = qkv_row_stride;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.q_w = q_norm_weight;
  a.k_w = k_norm_weight;
  a.w_dtype = norm_weight_dtype;
  a.eps = eps;
  a.cos_sin = cos_sin_cache;
  a.cs_dtype = cos_sin_dtype;
  a.max_position = max_position;
  a.positions = positions;
  a.q_out = q_out;
  a.k_out = k_out;
  a.out_dtype = out_dtype;
  a.k_cache = reinterpret_cast<char*>(k_cache);
  a.v_cache = reinterpret_cast<char*>(v_cache);
  a.cache_dtype = cache_dtype;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.calibrate = (flags & MKV_APPEND_CALIBRATE_SENTINEL) ? 1 : 0;
  a.slot_mapping = slot_mapping;
  a.num_slots = num_blocks * (int64_t)block_size;

  const int hpi = kWave / (head_dim / 16);
  const int64_t items = num_tokens * (int64_t)((num_heads + hpi - 1) / hpi + 2 * ((num_kv_heads + hpi - 1) / hpi));
  const dim3 grid((unsigned)((items + kProdWaves - 1) / kProdWaves));
  const dim3 block(kProdWaves * kWave);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define MKV_PROD(IDT, MODE) hipLaunchKernelGGL((qkv_producer_kernel<IDT, MODE>), grid, block, 0, s, a)
#define MKV_PROD_MODES(IDT)                                        \
  switch (mode) {                                                  \
    case kCacheCopy: MKV_PROD(IDT, kCacheCopy); break;             \
    case kCacheFp8Tensor: MKV_PROD(IDT, kCacheFp8Tensor); break;   \
    case kCacheFp8Token: MKV_PROD(IDT, kCacheFp8Token); break;     \
    default: MKV_PROD(IDT, kCacheI8Token); break;                  \
  }
  switch (in_dtype) {
    case MKV_DTYPE_F32: MKV_PROD_MODES(MKV_DTYPE_F32); break;
    case MKV_DTYPE_BF16: MKV_PROD_MODES(MKV_DTYPE_BF16); break;
    default: MKV_PROD_MODES(MKV_DTYPE_F16); break;
  }
#undef MKV_PROD_MODES
#undef MKV_PROD
  return (int)hipGetLastError();
}
