// Shared device-side helpers for the gfx950 KV-cache kernels: element
// conversions, the OCP e4m3fn codec, MFMA operand types and the block-table
// gather (K4) that the append, decode and prefill kernels all use.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mkv.h"

#define MKV_DEV __device__ __forceinline__

namespace mkv {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kFp8Max = 448.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

template <int DT>
struct DTypeInfo;
template <>
struct DTypeInfo<MKV_DTYPE_F32> {
  static constexpr int kBytes = 4;
};
template <>
struct DTypeInfo<MKV_DTYPE_BF16> {
  static constexpr int kBytes = 2;
};
template <>
struct DTypeInfo<MKV_DTYPE_F16> {
  static constexpr int kBytes = 2;
};
template <>
struct DTypeInfo<MKV_DTYPE_FP8E4M3> {
  static constexpr int kBytes = 1;
};
template <>
struct DTypeInfo<MKV_DTYPE_I8> {
  static constexpr int kBytes = 1;
};

// KV formats of the attention kernels that carry one fp32 scale per (token,
// KV head) in a tensor beside the pool.  These are template codes of the
// kernels, not ABI values: the C ABI names them by (dtype, scale mode).
constexpr int kKvFp8PerToken = 0x100 | MKV_DTYPE_FP8E4M3;
constexpr int kKvI8PerToken = 0x100 | MKV_DTYPE_I8;
template <>
struct DTypeInfo<kKvFp8PerToken> {
  static constexpr int kBytes = 1;
};
template <>
struct DTypeInfo<kKvI8PerToken> {
  static constexpr int kBytes = 1;
};
template <int KV_DT>
constexpr bool kPerTokenScale = KV_DT == kKvFp8PerToken || KV_DT == kKvI8PerToken;

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16 <-> f32 is done on the bit pattern; f32 -> bf16
// and f32 -> f16 round to nearest even like torch's Tensor.to().
// ---------------------------------------------------------------------------
MKV_DEV float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

MKV_DEV uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN (torch's canonical)
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

MKV_DEV float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

MKV_DEV uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Round an fp32 value to the precision of dtype DT and return it as fp32.
MKV_DEV float round_to_dtype(float f, int dt) {
  if (dt == MKV_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(f));
  if (dt == MKV_DTYPE_F16) return f16_bits_to_f32(f32_to_f16_bits(f));
  return f;
}

// ---------------------------------------------------------------------------
// OCP e4m3fn codec (the native fp8 format of gfx950's conversion units).
// ---------------------------------------------------------------------------

// torch.clamp(x, -448, 448) semantics: NaN passes through unchanged.
MKV_DEV float clamp_fp8_range(float v) {
  v = (v < -kFp8Max) ? -kFp8Max : v;
  v = (v > kFp8Max) ? kFp8Max : v;
  return v;
}

// Four fp32 values (already within +-448 or NaN) -> four e4m3fn bytes packed
// little-endian, rounding to nearest even (v_cvt_pk_fp8_f32).  A NaN input
// gives a NaN byte (low 7 bits 0x7f) whose sign is the converter's own;
// callers that need a particular NaN sign overwrite bit 7.
MKV_DEV uint32_t pack_fp8x4(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  return w;
}

// Sign of the NaN that an IEEE fp32 division x / s yields on the host CPU
// (x86 SSE, where torch's reference cast runs): a NaN operand is returned
// quieted with its sign (x first, then s); an invalid operation (0/0,
// inf/inf) returns the default NaN, whose sign bit is set.  The GPU divide
// returns a positive canonical NaN instead, so the quantiser restores this
// sign explicitly.  Returns 0 when x / s is not NaN.
MKV_DEV uint32_t div_nan_sign(float x, float s, float q) {
  if (q == q) return 0u;
  if (x != x) return __float_as_uint(x) >> 31;
  if (s != s) return __float_as_uint(s) >> 31;
  return 1u;
}

// The quantiser's scale with its reciprocal in fp64.  x / s correctly
// rounded to fp32 equals x * (1/s in fp64) rounded to fp32 for every fp32 x
// and s whose quotient is a normal fp32 number (smaller quotients become
// e4m3fn zero either way): the fp64 product is within 2^-52 (relative) of
// x / s, while a quotient of two 24-bit numbers is either an fp32 number or
// at least 2^-49 (relative) away from every midpoint between fp32 numbers
// (x - m s is a nonzero multiple of 2^-49 m s for a 25-bit midpoint m), so
// both round to the same fp32 value.  One fp64 product replaces the fp32
// division's refinement sequence.
struct Fp8Quant {
  float scale;
  double rcp;
};
MKV_DEV Fp8Quant fp8_quant(float scale) { return Fp8Quant{scale, 1.0 / (double)scale}; }

// Four fp32 values -> four e4m3fn bytes with the per-tensor quantiser's
// semantics: IEEE fp32 divide by the scale (correctly rounded, as above),
// torch.clamp to +-448 (NaN passes), round to nearest even.  NaN bytes keep
// the converter's S.1111.111 payload with the sign of the host's NaN
// (div_nan_sign), so the bytes equal torch's CPU cast.
MKV_DEV uint32_t quantize4_fp8(const float* x, const Fp8Quant& q) {
  float v[4];
  bool nan = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float qv = (float)((double)x[j] * q.rcp);
    nan |= qv != qv;
    v[j] = clamp_fp8_range(qv);
  }
  uint32_t w = pack_fp8x4(v[0], v[1], v[2], v[3]);
  if (nan) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (v[j] != v[j]) w = (w & ~(0x80u << (8 * j))) | (div_nan_sign(x[j], q.scale, v[j]) << (8 * j + 7));
  }
  return w;
}

MKV_DEV u32x4 quantize16_fp8(const float (&x)[16], const Fp8Quant& q) {
  return u32x4{quantize4_fp8(x, q), quantize4_fp8(x + 4, q), quantize4_fp8(x + 8, q), quantize4_fp8(x + 12, q)};
}

// INT8 code of x for the per-token-head quantiser: y = x * inv (inv =
// 1 / scale), rounded half away from zero, clamped to [-128, 127] with
// maxNum / minNum (a NaN becomes -128), truncated.
MKV_DEV uint32_t quantize_i8(float xv, float inv) {
  // (the product is rounded on its own, as in the reference: hipcc
  // compiles with -ffp-contract=fast, which could fuse it into the +-0.5
  // as one FMA with a single rounding; the empty asm keeps it apart)
  float y = xv * inv;
  asm volatile("" : "+v"(y));
  y = y >= 0.0f ? y + 0.5f : y - 0.5f;
  y = fminf(fmaxf(y, -128.0f), 127.0f);
  return (uint32_t)((int)y & 0xff);
}

MKV_DEV uint32_t quantize4_i8(const float* x, float inv) {
  return quantize_i8(x[0], inv) | (quantize_i8(x[1], inv) << 8) | (quantize_i8(x[2], inv) << 16) |
         (quantize_i8(x[3], inv) << 24);
}

MKV_DEV u32x4 quantize16_i8(const float (&x)[16], float inv) {
  return u32x4{quantize4_i8(x, inv), quantize4_i8(x + 4, inv), quantize4_i8(x + 8, inv),
               quantize4_i8(x + 12, inv)};
}

// Per-token-head scales from a head's amax (NaN elements excluded):
// FP8 amax / 448, or 1 for an all-zero head; INT8 max(amax / 127, 1e-6).
MKV_DEV float fp8_head_scale(float amax) { return amax > 0.0f ? amax / kFp8Max : 1.0f; }
MKV_DEV float i8_head_scale(float amax) { return fmaxf(amax / 127.0f, 1e-6f); }

// Two e4m3fn bytes (low or high half-word of w) -> exact fp16 pair.
template <bool kHi>
MKV_DEV f16x2 fp8x2_to_f16x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, kHi);
}

// Two e4m3fn bytes (low or high half-word of w) -> exact bf16 pair.
template <bool kHi>
MKV_DEV bf16x2 fp8x2_to_bf16x2(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, kHi);
}

// Two e4m3fn bytes -> exact fp32 pair.
template <bool kHi>
MKV_DEV f32x2 fp8x2_to_f32x2(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(w, kHi);
}

// ---------------------------------------------------------------------------
// Byte / half-word shuffles used to transpose K/V sub-tiles in registers.
// __builtin_amdgcn_perm(a, b, sel): result byte k = byte sel[k] of the 8-byte
// value {b (bytes 0-3), a (bytes 4-7)}.
// ---------------------------------------------------------------------------
MKV_DEV uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
  return __builtin_amdgcn_perm(a, b, sel);
}

// 4x4 byte transpose: rows r0..r3 (one dword each) -> columns c0..c3 where
// byte k of column j is byte j of row k.
MKV_DEV void transpose_bytes_4x4(uint32_t r0, uint32_t r1, uint32_t r2,
                                 uint32_t r3, uint32_t& c0, uint32_t& c1,
                                 uint32_t& c2, uint32_t& c3) {
  const uint32_t t01l = perm(r1, r0, 0x05010400u);  // r0.0 r1.0 r0.1 r1.1
  const uint32_t t01h = perm(r1, r0, 0x07030602u);  // r0.2 r1.2 r0.3 r1.3
  const uint32_t t23l = perm(r3, r2, 0x05010400u);
  const uint32_t t23h = perm(r3, r2, 0x07030602u);
  c0 = perm(t23l, t01l, 0x05040100u);
  c1 = perm(t23l, t01l, 0x07060302u);
  c2 = perm(t23h, t01h, 0x05040100u);
  c3 = perm(t23h, t01h, 0x07060302u);
}

// Low half-words of (a, b) -> {a.lo, b.lo}; high half-words -> {a.hi, b.hi}.
MKV_DEV uint32_t pack_lo16(uint32_t a, uint32_t b) { return perm(b, a, 0x05040100u); }
MKV_DEV uint32_t pack_hi16(uint32_t a, uint32_t b) { return perm(b, a, 0x07060302u); }

// Two int8 codes (bytes 0-1 of w, or bytes 2-3 with kHi) -> exact bf16 pair:
// an integer of magnitude <= 128 has at most 8 significant bits, so the upper
// half-word of its fp32 value is that value in bf16.
template <bool kHi>
MKV_DEV bf16x2 i8x2_to_bf16x2(uint32_t w) {
  const float a = (float)(int8_t)(w >> (kHi ? 16 : 0));
  const float b = (float)(int8_t)(w >> (kHi ? 24 : 8));
  return __builtin_bit_cast(bf16x2, pack_hi16(__float_as_uint(a), __float_as_uint(b)));
}

// Two int8 codes (bytes 0-1 of w, or bytes 2-3 with kHi) -> exact fp16 pair
// (an integer of magnitude <= 128 is exact in fp16; the truncating pack
// changes no exact value).
template <bool kHi>
MKV_DEV f16x2 i8x2_to_f16x2(uint32_t w) {
  const float a = (float)(int8_t)(w >> (kHi ? 16 : 0));
  const float b = (float)(int8_t)(w >> (kHi ? 24 : 8));
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// Value of lane N of this lane's 16-lane row (DPP row broadcast).
template <int N>
MKV_DEV float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + N, 0xf, 0xf, true));
}

// ---------------------------------------------------------------------------
// Global memory access helpers.
// ---------------------------------------------------------------------------
MKV_DEV u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
MKV_DEV u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
MKV_DEV void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// 32 consecutive q elements (fp32, bf16 or fp16; element offset off a
// multiple of 8) as fp32, in two steps: q32_issue issues every load of the
// slice (4 for 16-bit q, 8 for fp32) and q32_convert, called once they are
// needed, converts them, so the loads share one round trip and other loads
// can go out in between (a load, wait and convert per 8 elements took four
// round trips in a row).
struct Q32Raw {
  u32x4 r[8];
};
MKV_DEV void q32_issue(const void* q, int dt, int64_t off, Q32Raw& w) {
  if (dt == MKV_DTYPE_F32) {
    const float* p = reinterpret_cast<const float*>(q) + off;
#pragma unroll
    for (int i = 0; i < 8; ++i) w.r[i] = ld16(p + 4 * i);
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(q) + off;
#pragma unroll
    for (int i = 0; i < 4; ++i) w.r[i] = ld16(p + 8 * i);
  }
}
MKV_DEV void q32_convert(int dt, const Q32Raw& w, float* x) {
  if (dt == MKV_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * i + j] = __uint_as_float(w.r[i][j]);
  } else if (dt == MKV_DTYPE_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * i + 2 * j] = bf16_bits_to_f32(w.r[i][j] & 0xffffu);
        x[8 * i + 2 * j + 1] = bf16_bits_to_f32(w.r[i][j] >> 16);
      }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * i + 2 * j] = f16_bits_to_f32(w.r[i][j] & 0xffffu);
        x[8 * i + 2 * j + 1] = f16_bits_to_f32(w.r[i][j] >> 16);
      }
  }
}
MKV_DEV void load_q32(const void* q, int dt, int64_t off, float* x) {
  Q32Raw w;
  q32_issue(q, dt, off, w);
  q32_convert(dt, w, x);
}

// Non-temporal 16-byte load for streamed-once KV bytes.
MKV_DEV u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
MKV_DEV u32x2 ld8_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

MKV_DEV int64_t load_index(const void* p, int64_t i, int is_i64) {
  return is_i64 ? reinterpret_cast<const int64_t*>(p)[i]
                : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

MKV_DEV int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A wave-uniform fp32 that no kernel writes (e.g. a per-tensor scale), read
// through the constant address space so that it becomes a scalar load: a
// vector load consumed at once would make the wave wait for every load it has
// in flight.
MKV_DEV float load_uniform_f32(const float* p) {
  typedef const float __attribute__((address_space(4))) const_f32;
  return *((const_f32*)p);
}

// ---------------------------------------------------------------------------
// K4: block-table gather.  Logical token t of sequence b lives in physical
// block block_tables[b, t >> log2(bs)] at offset t & (bs - 1).  An entry of -1
// (or any entry outside the pool) marks the block absent; the caller masks
// such tokens.  Offsets are 64-bit: a bf16 pool of a few thousand 256-token
// blocks already exceeds 2^31 bytes.
// ---------------------------------------------------------------------------
struct PagedIndex {
  const int32_t* block_tables;
  int64_t bt_stride;
  int max_blocks;
  int64_t num_blocks;
  int bs_log2;
  int64_t row_elems;  // num_kv_heads * head_dim: elements per token row

  // Physical block of logical block `blk` of sequence `seq`, or -1.  The table
  // is read through the constant address space (no kernel writes it): with a
  // wave-uniform index this becomes a scalar load, which is counted apart from
  // the vector-memory counter, so looking up the next tile never waits for the
  // K/V loads already in flight.
  MKV_DEV int64_t physical_block(int seq, int64_t blk) const {
    if (blk < 0 || blk >= max_blocks) return -1;
    typedef const int32_t __attribute__((address_space(4))) const_i32;
    const int64_t p = ((const_i32*)block_tables)[(int64_t)seq * bt_stride + blk];
    return (p >= 0 && p < num_blocks) ? p : -1;
  }

  // Element offset of token row (phys, t) in the pool (head 0, dim 0).
  MKV_DEV int64_t row_offset(int64_t phys, int64_t t) const {
    return ((phys << bs_log2) + (t & ((int64_t(1) << bs_log2) - 1))) * row_elems;
  }
};

// ---------------------------------------------------------------------------
// Head pairing (head_dim 64).  The attention kernels work on 128-element
// head rows.  KV heads 2v and 2v+1 of a head_dim-64 cache are adjacent
// 64-element segments of a token row, so the kernels read them as one
// 128-element segment, KV head v of the kernel, whose group holds the 2G
// query heads 2vG .. 2vG+2G-1 (those of KV head 2v, then those of 2v+1).
// Query head j of that group takes dims 64*hi(j) .. +63 of the segment,
// hi(j) = (j >= G): its q is zero on the other half, so its scores are
// exact, and only its own half of the output is stored.  Pool, block tables
// and every K/V tile load are those of a head_dim-128 pool with Hkv/2 KV
// heads; q, the output and the per-token-head scales are addressed with the
// caller's shape.
// ---------------------------------------------------------------------------
template <bool PAIR>
constexpr int kQDim = PAIR ? 64 : 128;

// q slice of lane (c, kg): dims 32kg .. 32kg+31 of head c of the kernel's
// group.  Returns false for a lane that holds zeros (a padding head, or the
// other half of a paired head); dim0 = the slice's first element in q's head
// row.
template <bool PAIR>
MKV_DEV bool q_slice(int group, int c, int kg, int& dim0) {
  if constexpr (PAIR) {
    const bool hi = c >= (group >> 1);
    dim0 = 32 * (kg & 1);
    return c < group && (kg >> 1) == (hi ? 1 : 0);
  } else {
    dim0 = 32 * kg;
    return c < group;
  }
}

// Output columns 8c .. 8c+7 of head h of the kernel's group: whether they
// belong to the head's own output, and their first element in its output
// row.
template <bool PAIR>
MKV_DEV bool out_cols(int group, int h, int c, int& col0) {
  if constexpr (PAIR) {
    const bool hi = h >= (group >> 1);
    col0 = 8 * c - (hi ? 64 : 0);
    return (c >= 8) == hi;
  } else {
    col0 = 8 * c;
    return true;
  }
}

}  // namespace mkv
