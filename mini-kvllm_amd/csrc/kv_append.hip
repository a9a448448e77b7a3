// K1: slot-mapped KV append with optional fused quantisation (per-tensor FP8,
// per-token-head FP8 or INT8), plus the device-side per-tensor FP8
// calibration.
//
// Reference semantics: store_kvcache (attention.py:67-108, kernel :7-64),
// store_kvcache_fp8 (attention.py:281-333, kernel :118-191: per-tensor branch
// :183-189, per-token-head branch :166-181), store_kvcache_int8
// (attention.py:246-276, kernel :194-243) and the calibrate-once rule
// (attention.py:308-323).
//
// Design: one wavefront per token row.  A row (all KV heads of one token) is
// num_kv_heads * head_dim contiguous elements in both the input and the pool,
// so a wave streams it with 16-byte loads and 16-byte stores: for bf16 -> fp8
// each lane reads 32 bytes and writes 16 bytes, a whole 1 KiB pool row per
// wave instruction.  The reference launches one program per (token, head).
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kAppendWaves = 4;  // token rows per 256-thread workgroup
constexpr int kElemsPerLane = 16;

template <int IN_DT>
MKV_DEV void load16_as_f32(const void* row, int64_t e, float (&x)[16]) {
  if constexpr (IN_DT == MKV_DTYPE_F32) {
    const float* p = reinterpret_cast<const float*>(row) + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 w = ld16(p + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * i + j] = __uint_as_float(w[j]);
    }
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row) + e;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      u32x4 w = ld16(p + 8 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (IN_DT == MKV_DTYPE_BF16) {
          x[8 * i + 2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
          x[8 * i + 2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
        } else {
          x[8 * i + 2 * j] = f16_bits_to_f32(w[j] & 0xffffu);
          x[8 * i + 2 * j + 1] = f16_bits_to_f32(w[j] >> 16);
        }
      }
    }
  }
}

// load16_as_f32 with non-temporal loads: each input row is read once.
template <int IN_DT>
MKV_DEV void load16_as_f32_stream(const void* row, int64_t e, float (&x)[16]) {
  if constexpr (IN_DT == MKV_DTYPE_F32) {
    const float* p = reinterpret_cast<const float*>(row) + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 w = ld16_stream(p + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * i + j] = __uint_as_float(w[j]);
    }
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row) + e;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 w = ld16_stream(p + 8 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * i + 2 * j] = IN_DT == MKV_DTYPE_BF16 ? bf16_bits_to_f32(w[j] & 0xffffu) : f16_bits_to_f32(w[j] & 0xffffu);
        x[8 * i + 2 * j + 1] = IN_DT == MKV_DTYPE_BF16 ? bf16_bits_to_f32(w[j] >> 16) : f16_bits_to_f32(w[j] >> 16);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Per-tensor calibration: amax over every row (slot -1 rows included), then
// scale = round_in(max(amax, round_in(1e-8)) / 448) for each tensor whose
// scale still holds the 1.0 sentinel.  The last workgroup to finish computes
// the scales and returns the workspace to zero, so the kernel is safe to
// record in a graph and needs no memset.
// ---------------------------------------------------------------------------
constexpr int kCalThreads = 256;

template <int IN_DT>
MKV_DEV float row_chunk_absmax(const char* row, int64_t e) {
  float x[16];
  load16_as_f32<IN_DT>(row, e, x);
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float a = fabsf(x[i]);
    // NaN must win, as in torch.amax: compare on the bit pattern.
    m = __uint_as_float(max(__float_as_uint(m), __float_as_uint(a)));
  }
  return m;
}

MKV_DEV uint32_t block_max_u32(uint32_t v, uint32_t* smem) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) smem[w] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kCalThreads / kWave; ++i) v = max(v, smem[i]);
  }
  return v;
}

// The calibrated scale from the amax bit pattern (a NaN amax propagates).
template <int IN_DT>
MKV_DEV float calibrated_scale(uint32_t amax_bits) {
  const float lo = round_to_dtype(1e-8f, IN_DT);
  float a = __uint_as_float(amax_bits);
  a = (a < lo) ? lo : a;  // clamp(min=1e-8); NaN propagates
  return round_to_dtype(a / kFp8Max, IN_DT);
}

// A scale that still holds the 1.0 sentinel when the append runs: the wave
// reads every row (slot -1 rows included) and derives the calibrated scale
// itself, exactly as fp8_calibrate_kernel would, and writes it back.  Every
// wave that sees the sentinel computes the same value, so a wave that reads
// the scale after another one wrote it quantises identically.  Only reached
// when calibration was not run first (the Python layer runs it on a scale
// tensor's first use) or produced exactly 1.0; it is slow (every wave reads
// the whole input) and meant to keep the reference's semantics in those
// cases, not to be the calibration path.
template <int IN_DT>
MKV_DEV float calibrate_in_wave(const void* x, int64_t stride, int64_t num_tokens, int64_t row_elems,
                                float* scale) {
  constexpr int kInBytes = DTypeInfo<IN_DT>::kBytes;
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t m = 0;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const char* row = reinterpret_cast<const char*>(x) + t * stride * kInBytes;
    for (int64_t e = (int64_t)lane * kElemsPerLane; e < row_elems; e += kWave * kElemsPerLane)
      m = max(m, __float_as_uint(row_chunk_absmax<IN_DT>(row, e)));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
  const float sc = calibrated_scale<IN_DT>(m);
  if (lane == 0) *scale = sc;
  return sc;
}

template <int IN_DT, bool FP8>
__global__ __launch_bounds__(kAppendWaves* kWave) void kv_append_kernel(
    const void* __restrict__ key, int64_t key_stride,
    const void* __restrict__ value, int64_t value_stride,
    void* __restrict__ k_cache, void* __restrict__ v_cache,
    const int64_t* __restrict__ slot_mapping, int64_t num_tokens,
    int64_t row_elems, int64_t num_slots, float* k_scale, float* v_scale, int calibrate) {
  constexpr int kInBytes = DTypeInfo<IN_DT>::kBytes;
  constexpr int kOutBytes = FP8 ? 1 : kInBytes;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = (int64_t)blockIdx.x * kAppendWaves + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  float ks = 0.0f, vs = 0.0f;
  if constexpr (FP8) {
    ks = *k_scale;
    vs = *v_scale;
    // before the slot test: a padding row still calibrates (all rows count)
    if (calibrate && ks == 1.0f)
      ks = calibrate_in_wave<IN_DT>(key, key_stride, num_tokens, row_elems, k_scale);
    if (calibrate && vs == 1.0f)
      vs = calibrate_in_wave<IN_DT>(value, value_stride, num_tokens, row_elems, v_scale);
  }
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;  // -1 = padding: skip

  const char* krow = reinterpret_cast<const char*>(key) + t * key_stride * kInBytes;
  const char* vrow = reinterpret_cast<const char*>(value) + t * value_stride * kInBytes;
  char* kdst = reinterpret_cast<char*>(k_cache) + slot * row_elems * kOutBytes;
  char* vdst = reinterpret_cast<char*>(v_cache) + slot * row_elems * kOutBytes;

  if constexpr (FP8) {
    const Fp8Quant kq = fp8_quant(ks), vq = fp8_quant(vs);
    // K and V are loaded before either is quantised (one memory round trip
    // per row, not two), inputs and pool rows bypass the caches
    // (non-temporal), and the divide by the scale is one fp64 product
    // (fp8_quant): 65,536 tokens in ~77 us (5.2 TB/s of K/V reads and code
    // writes, the copy append's rate) against ~80 us with the fp32 division.
    for (int64_t e = (int64_t)lane * kElemsPerLane; e < row_elems; e += kWave * kElemsPerLane) {
      float xk[16], xv[16];
      load16_as_f32_stream<IN_DT>(krow, e, xk);
      load16_as_f32_stream<IN_DT>(vrow, e, xv);
      __builtin_nontemporal_store(quantize16_fp8(xk, kq), reinterpret_cast<u32x4*>(kdst + e));
      __builtin_nontemporal_store(quantize16_fp8(xv, vq), reinterpret_cast<u32x4*>(vdst + e));
    }
  } else {
    // Plain copy in 16-byte units.
    const int64_t row_bytes = row_elems * kInBytes;
    for (int64_t o = (int64_t)lane * 16; o < row_bytes; o += kWave * 16) {
      const u32x4 kv = ld16_stream(krow + o);
      const u32x4 vv = ld16_stream(vrow + o);
      __builtin_nontemporal_store(kv, reinterpret_cast<u32x4*>(kdst + o));
      __builtin_nontemporal_store(vv, reinterpret_cast<u32x4*>(vdst + o));
    }
  }
}

template <int IN_DT>
__global__ __launch_bounds__(kCalThreads) void fp8_calibrate_kernel(
    const void* __restrict__ key, int64_t key_stride,
    const void* __restrict__ value, int64_t value_stride, int64_t num_tokens,
    int64_t row_elems, float* __restrict__ k_scale, float* __restrict__ v_scale,
    uint32_t* __restrict__ ws) {
  constexpr int kInBytes = DTypeInfo<IN_DT>::kBytes;
  __shared__ uint32_t smem[2 * kCalThreads / kWave];
  __shared__ bool is_last;
  const bool need_k = (*k_scale == 1.0f);
  const bool need_v = (*v_scale == 1.0f);
  if (!need_k && !need_v) return;  // uniform for the whole grid

  const int64_t chunks_per_row = row_elems / 16;
  const int64_t total = num_tokens * chunks_per_row;
  uint32_t km = 0, vm = 0;
  for (int64_t c = (int64_t)blockIdx.x * kCalThreads + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * kCalThreads) {
    const int64_t t = c / chunks_per_row;
    const int64_t e = (c - t * chunks_per_row) * 16;
    if (need_k) {
      const char* row = reinterpret_cast<const char*>(key) + t * key_stride * kInBytes;
      km = max(km, __float_as_uint(row_chunk_absmax<IN_DT>(row, e)));
    }
    if (need_v) {
      const char* row = reinterpret_cast<const char*>(value) + t * value_stride * kInBytes;
      vm = max(vm, __float_as_uint(row_chunk_absmax<IN_DT>(row, e)));
    }
  }
  km = block_max_u32(km, smem);
  __syncthreads();
  vm = block_max_u32(vm, smem + kCalThreads / kWave);
  if (threadIdx.x == 0) {
    if (need_k) atomicMax(&ws[0], km);
    if (need_v) atomicMax(&ws[1], vm);
    __threadfence();
    const uint32_t done = atomicAdd(&ws[2], 1u);
    is_last = (done == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last || threadIdx.x != 0) return;
  __threadfence();
  const float lo = round_to_dtype(1e-8f, IN_DT);
  if (need_k) {
    float a = __uint_as_float(atomicAdd(&ws[0], 0u));
    a = (a < lo) ? lo : a;  // clamp(min=1e-8); NaN propagates
    *k_scale = round_to_dtype(a / kFp8Max, IN_DT);
  }
  if (need_v) {
    float a = __uint_as_float(atomicAdd(&ws[1], 0u));
    a = (a < lo) ? lo : a;
    *v_scale = round_to_dtype(a / kFp8Max, IN_DT);
  }
  atomicExch(&ws[0], 0u);
  atomicExch(&ws[1], 0u);
  atomicExch(&ws[2], 0u);
}

// ---------------------------------------------------------------------------
// Per-token-head quantisation (FP8 e4m3fn or INT8): every (token, KV head)
// gets its own fp32 scale from the amax of its head_dim elements.  A lane
// holds 16 consecutive elements, so one head is D/16 adjacent lanes and its
// amax is an xor-shuffle reduction over them (D a power of two, 16..1024).
// ---------------------------------------------------------------------------

// amax of |x| over the lane's 16 elements, NaN ignored (maxNum), then over
// the `group` lanes of the head.
template <int IN_DT>
MKV_DEV float head_amax(const void* row, int64_t e, int group, float (&x)[16]) {
  load16_as_f32<IN_DT>(row, e, x);
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(x[i]));
  for (int off = 1; off < group; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
  return m;
}

template <int IN_DT, bool INT8>
MKV_DEV void quantize_head_chunk(const char* row, char* dst, float* scales, int64_t e, int group,
                                 int head_dim, int lane) {
  float x[16];
  const float amax = head_amax<IN_DT>(row, e, group, x);
  u32x4 q;
  float scale;
  if constexpr (INT8) {
    scale = i8_head_scale(amax);
    q = quantize16_i8(x, 1.0f / scale);
  } else {
    scale = fp8_head_scale(amax);
    q = quantize16_fp8(x, fp8_quant(scale));
  }
  st16(dst + e, q);
  if ((lane & (group - 1)) == 0) scales[e / head_dim] = scale;
}

template <int IN_DT, bool INT8>
__global__ __launch_bounds__(kAppendWaves* kWave) void kv_append_per_token_head_kernel(
    const void* __restrict__ key, int64_t key_stride,
    const void* __restrict__ value, int64_t value_stride,
    void* __restrict__ k_cache, void* __restrict__ v_cache,
    float* __restrict__ k_scale, float* __restrict__ v_scale,
    const int64_t* __restrict__ slot_mapping, int64_t num_tokens,
    int num_kv_heads, int head_dim, int64_t num_slots) {
  constexpr int kInBytes = DTypeInfo<IN_DT>::kBytes;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = (int64_t)blockIdx.x * kAppendWaves + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;  // -1 = padding: skip

  const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
  const int group = head_dim / kElemsPerLane;  // lanes per head
  const char* krow = reinterpret_cast<const char*>(key) + t * key_stride * kInBytes;
  const char* vrow = reinterpret_cast<const char*>(value) + t * value_stride * kInBytes;
  char* kdst = reinterpret_cast<char*>(k_cache) + slot * row_elems;
  char* vdst = reinterpret_cast<char*>(v_cache) + slot * row_elems;
  float* ks = k_scale + slot * num_kv_heads;
  float* vs = v_scale + slot * num_kv_heads;
  // Whole heads per iteration (a head spans group <= 64 lanes, aligned), so
  // the lanes of one head are always active together.
  for (int64_t e = (int64_t)lane * kElemsPerLane; e < row_elems; e += kWave * kElemsPerLane) {
    quantize_head_chunk<IN_DT, INT8>(krow, kdst, ks, e, group, head_dim, lane);
    quantize_head_chunk<IN_DT, INT8>(vrow, vdst, vs, e, group, head_dim, lane);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_kv_append(const void* key, int64_t key_row_stride, const void* value,
                             int64_t value_row_stride, void* k_cache, void* v_cache,
                             const int64_t* slot_mapping, int64_t num_tokens, int num_kv_heads,
                             int head_dim, int block_size, int64_t num_blocks, int in_dtype,
                             int cache_dtype, float* k_scale, float* v_scale, int flags,
                             void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0)
    return MKV_ERR_BAD_SHAPE;
  if (num_tokens == 0) return MKV_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return MKV_ERR_NULL_POINTER;
  const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
  if (row_elems % 16 != 0) return MKV_ERR_BAD_SHAPE;
  if (in_dtype != MKV_DTYPE_F32 && in_dtype != MKV_DTYPE_BF16 && in_dtype != MKV_DTYPE_F16)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  const bool fp8 = (cache_dtype == MKV_DTYPE_FP8E4M3);
  if (!fp8 && cache_dtype != in_dtype) return MKV_ERR_UNSUPPORTED_DTYPE;
  if (fp8 && (!k_scale || !v_scale)) return MKV_ERR_NULL_POINTER;
  if (flags & ~MKV_APPEND_CALIBRATE_SENTINEL) return MKV_ERR_BAD_SHAPE;
  const int calibrate = (flags & MKV_APPEND_CALIBRATE_SENTINEL) ? 1 : 0;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return MKV_ERR_BAD_STRIDE;
  const int in_bytes = (in_dtype == MKV_DTYPE_F32) ? 4 : 2;
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) ||
      (key_row_stride * in_bytes) % 16 != 0 || (value_row_stride * in_bytes) % 16 != 0)
    return MKV_ERR_MISALIGNED;

  const int64_t num_slots = num_blocks * (int64_t)block_size;
  const dim3 grid((unsigned)((num_tokens + kAppendWaves - 1) / kAppendWaves));
  const dim3 block(kAppendWaves * kWave);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define MKV_APPEND_LAUNCH(IDT, F8)                                                            \
  hipLaunchKernelGGL((kv_append_kernel<IDT, F8>), grid, block, 0, s, key, key_row_stride,      \
                     value, value_row_stride, k_cache, v_cache, slot_mapping, num_tokens,      \
                     row_elems, num_slots, k_scale, v_scale, calibrate)
  switch (in_dtype) {
    case MKV_DTYPE_F32:
      if (fp8) MKV_APPEND_LAUNCH(MKV_DTYPE_F32, true); else MKV_APPEND_LAUNCH(MKV_DTYPE_F32, false);
      break;
    case MKV_DTYPE_BF16:
      if (fp8) MKV_APPEND_LAUNCH(MKV_DTYPE_BF16, true); else MKV_APPEND_LAUNCH(MKV_DTYPE_BF16, false);
      break;
    default:
      if (fp8) MKV_APPEND_LAUNCH(MKV_DTYPE_F16, true); else MKV_APPEND_LAUNCH(MKV_DTYPE_F16, false);
      break;
  }
#undef MKV_APPEND_LAUNCH
  return (int)hipGetLastError();
}

extern "C" size_t mkv_fp8_calibrate_workspace_size(void) { return 4 * sizeof(uint32_t); }

extern "C" int mkv_fp8_calibrate_per_tensor(const void* key, int64_t key_row_stride,
                                            const void* value, int64_t value_row_stride,
                                            int64_t num_tokens, int row_elems, int in_dtype,
                                            float* k_scale, float* v_scale, void* workspace,
                                            void* stream) {
  if (num_tokens < 0 || row_elems <= 0 || row_elems % 16 != 0) return MKV_ERR_BAD_SHAPE;
  if (!k_scale || !v_scale || !workspace) return MKV_ERR_NULL_POINTER;
  if (num_tokens > 0 && (!key || !value)) return MKV_ERR_NULL_POINTER;
  if (in_dtype != MKV_DTYPE_F32 && in_dtype != MKV_DTYPE_BF16 && in_dtype != MKV_DTYPE_F16)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return MKV_ERR_BAD_STRIDE;
  const int in_bytes = (in_dtype == MKV_DTYPE_F32) ? 4 : 2;
  if ((num_tokens > 0 && (!aligned16(key) || !aligned16(value))) ||
      (key_row_stride * in_bytes) % 16 != 0 || (value_row_stride * in_bytes) % 16 != 0)
    return MKV_ERR_MISALIGNED;
  const int64_t chunks = num_tokens * (row_elems / 16);
  int64_t blocks = (chunks + kCalThreads * 4 - 1) / (kCalThreads * 4);
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* ws = reinterpret_cast<uint32_t*>(workspace);
#define MKV_CAL_LAUNCH(IDT)                                                                     \
  hipLaunchKernelGGL((fp8_calibrate_kernel<IDT>), dim3((unsigned)blocks), dim3(kCalThreads), 0, \
                     s, key, key_row_stride, value, value_row_stride, num_tokens,              \
                     (int64_t)row_elems, k_scale, v_scale, ws)
  switch (in_dtype) {
    case MKV_DTYPE_F32: MKV_CAL_LAUNCH(MKV_DTYPE_F32); break;
    case MKV_DTYPE_BF16: MKV_CAL_LAUNCH(MKV_DTYPE_BF16); break;
    default: MKV_CAL_LAUNCH(MKV_DTYPE_F16); break;
  }
#undef MKV_CAL_LAUNCH
  return (int)hipGetLastError();
}

extern "C" int mkv_kv_append_per_token_head(const void* key, int64_t key_row_stride,
                                            const void* value, int64_t value_row_stride,
                                            void* k_cache, void* v_cache, float* k_scale,
                                            float* v_scale, const int64_t* slot_mapping,
                                            int64_t num_tokens, int num_kv_heads, int head_dim,
                                            int block_size, int64_t num_blocks, int in_dtype,
                                            int cache_dtype, void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0)
    return MKV_ERR_BAD_SHAPE;
  if (head_dim < 16 || head_dim > 1024 || (head_dim & (head_dim - 1))) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  if (num_tokens == 0) return MKV_OK;
  if (!key || !value || !k_cache || !v_cache || !k_scale || !v_scale || !slot_mapping)
    return MKV_ERR_NULL_POINTER;
  if (in_dtype != MKV_DTYPE_F32 && in_dtype != MKV_DTYPE_BF16 && in_dtype != MKV_DTYPE_F16)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (cache_dtype != MKV_DTYPE_FP8E4M3 && cache_dtype != MKV_DTYPE_I8) return MKV_ERR_UNSUPPORTED_DTYPE;
  const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return MKV_ERR_BAD_STRIDE;
  const int in_bytes = (in_dtype == MKV_DTYPE_F32) ? 4 : 2;
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) ||
      (key_row_stride * in_bytes) % 16 != 0 || (value_row_stride * in_bytes) % 16 != 0)
    return MKV_ERR_MISALIGNED;

  const int64_t num_slots = num_blocks * (int64_t)block_size;
  const dim3 grid((unsigned)((num_tokens + kAppendWaves - 1) / kAppendWaves));
  const dim3 block(kAppendWaves * kWave);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool i8 = cache_dtype == MKV_DTYPE_I8;
#define MKV_PTH_LAUNCH(IDT, I8)                                                                  \
  hipLaunchKernelGGL((kv_append_per_token_head_kernel<IDT, I8>), grid, block, 0, s, key,          \
                     key_row_stride, value, value_row_stride, k_cache, v_cache, k_scale, v_scale, \
                     slot_mapping, num_tokens, num_kv_heads, head_dim, num_slots)
  switch (in_dtype) {
    case MKV_DTYPE_F32:
      if (i8) MKV_PTH_LAUNCH(MKV_DTYPE_F32, true); else MKV_PTH_LAUNCH(MKV_DTYPE_F32, false);
      break;
    case MKV_DTYPE_BF16:
      if (i8) MKV_PTH_LAUNCH(MKV_DTYPE_BF16, true); else MKV_PTH_LAUNCH(MKV_DTYPE_BF16, false);
      break;
    default:
      if (i8) MKV_PTH_LAUNCH(MKV_DTYPE_F16, true); else MKV_PTH_LAUNCH(MKV_DTYPE_F16, false);
      break;
  }
#undef MKV_PTH_LAUNCH
  return (int)hipGetLastError();
}
