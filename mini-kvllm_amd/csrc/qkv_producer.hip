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
// a full-prefill attention over fresh K/V.  The per-lane arithmetic (lane
// layout, norm, rotation, quantisation) lives in qkv_producer.hpp.
#include "qkv_producer.hpp"

namespace mkv {
namespace {

constexpr int kProdWaves = 4;

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
    float wkl[8] = {}, wkh[8] = {};
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
  float wl[8] = {}, wh[8] = {};
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
