// Device side of the fused producer (q/k RMSNorm + rotary embedding + KV
// append), shared by the producer kernel and the decode kernel that runs the
// producer's step for a decode batch before its attention: both compile the
// same arithmetic, so the two give the same bits.
//
// Reference: LayerNorm.rms_forward (layernorm.py:16-24), apply_rotary_pos_emb
// (rotary_embedding.py:4-26, :100-109), store_kvcache / store_kvcache_fp8 /
// store_kvcache_int8 (attention.py:255-333, :1654-1691).
//
// Lane layout: a head of D elements is D/16 lanes; lane m of a head holds
// elements [8m, 8m+8) and [D/2 + 8m, D/2 + 8m + 8), i.e. 8 rotary pairs, so
// the rotation is lane-local and only the norm's sum of squares is reduced
// across the head's lanes.
#pragma once
#include "mkv_device.hpp"

namespace mkv {
namespace {

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

// An fp32 product rounded on its own.  hipcc compiles with
// -ffp-contract=fast, which fuses a product into the sum that consumes it
// (one FMA, one rounding) whatever the source asks for (__fmul_rn is the
// plain operator, and `#pragma clang fp contract(off)` is not honoured); an
// empty asm statement on the product hides its origin from that fusion and
// emits nothing.
MKV_DEV float mul_rn(float x, float y) {
  float p = x * y;
  asm volatile("" : "+v"(p));
  return p;
}

// Norm (if a weight is given) and rotation of the lane's 8 + 8 elements x1
// (offsets 8m..) and x2 (D/2 + 8m..) of a q/k head, in fp32 after rounding
// to out_dtype: the value of the reference's rotated tensor.
//   norm:   y = round_in(x / sqrt(sum(x^2) / D + eps) * w)
//   rotary: o1 = y1 * cos - y2 * sin, o2 = y1 * sin + y2 * cos  (no FMA)
// (the head's D/16 lanes must run it together: the sum of squares is a
// shuffle reduction over them).  Every product that feeds a sum goes
// through mul_rn, so that it is rounded before the sum as in the reference.
MKV_DEV void norm_rope(const ProducerArgs& a, float (&x1)[8], float (&x2)[8], const void* w,
                       const float (&wl)[8], const float (&wh)[8], const float (&c)[8], const float (&s)[8],
                       int in_dt, float (&o1)[8], float (&o2)[8]) {
  if (w) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __fadd_rn(ss, __fadd_rn(mul_rn(x1[j], x1[j]), mul_rn(x2[j], x2[j])));
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
    o1[j] = round_to_dtype(__fsub_rn(mul_rn(x1[j], c[j]), mul_rn(x2[j], s[j])), a.out_dtype);
    o2[j] = round_to_dtype(__fadd_rn(mul_rn(x1[j], s[j]), mul_rn(x2[j], c[j])), a.out_dtype);
  }
}

// The lane's 8 + 8 elements of q/k head `head` (element offset of the head in
// the qkv row), normed and rotated (norm_rope).
MKV_DEV void produce_qk(const ProducerArgs& a, const char* row, int64_t head_off, const void* w,
                        const float (&wl)[8], const float (&wh)[8], const float (&c)[8],
                        const float (&s)[8], int m, int in_dt, float (&o1)[8], float (&o2)[8]) {
  const int half = a.head_dim / 2;
  const int eb = dtype_bytes(in_dt);
  float x1[8], x2[8];
  load8_f32(row + (head_off + 8 * m) * eb, in_dt, x1);
  load8_f32(row + (head_off + half + 8 * m) * eb, in_dt, x2);
  norm_rope(a, x1, x2, w, wl, wh, c, s, in_dt, o1, o2);
}

// 8 consecutive elements of dtype dt as raw words (16 bytes, 32 for fp32),
// for callers that issue the loads early and convert later; the second load
// reads the first 16 bytes again for 16-bit types, so the load sequence has
// no branch.
struct Raw8 {
  u32x4 w0, w1;
};
MKV_DEV Raw8 load_raw8(const void* p, int dt) {
  const char* q = reinterpret_cast<const char*>(p);
  return Raw8{ld16(q), ld16(dt == MKV_DTYPE_F32 ? q + 16 : q)};
}
// The elements of a Raw8 in fp32 (exact), as load8_f32 gives them (selects,
// not branches: arrays defined on two paths land in scratch memory).
MKV_DEV void raw8_f32(const Raw8& r, int dt, float (&x)[8]) {
  const bool f32 = dt == MKV_DTYPE_F32, bf = dt == MKV_DTYPE_BF16;
  float h[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = r.w0[j];
    h[2 * j] = bf ? bf16_bits_to_f32(w & 0xffffu) : f16_bits_to_f32(w & 0xffffu);
    h[2 * j + 1] = bf ? bf16_bits_to_f32(w >> 16) : f16_bits_to_f32(w >> 16);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[j] = f32 ? __uint_as_float(r.w0[j]) : h[j];
    x[4 + j] = f32 ? __uint_as_float(r.w1[j]) : h[4 + j];
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
  // (a row of the table is read either way, so no branch leaves the arrays
  // defined on two paths: that put them in scratch memory)
  const bool ok = pos >= 0 && pos < a.max_position;
  const int eb = dtype_bytes(a.cs_dtype);
  const char* row = reinterpret_cast<const char*>(a.cos_sin) + (ok ? pos : 0) * a.head_dim * eb;
  load8_f32(row + (8 * m) * eb, a.cs_dtype, c);
  load8_f32(row + (a.head_dim / 2 + 8 * m) * eb, a.cs_dtype, s);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    c[j] = ok ? c[j] : __builtin_nanf("");
    s[j] = ok ? s[j] : __builtin_nanf("");
  }
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

}  // namespace
}  // namespace mkv
