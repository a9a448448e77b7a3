// Fused row operations of the engine's decoder layer around the KV-cache
// path: residual add + RMSNorm, and SiLU-and-multiply.
//
// Reference: LayerNorm.rms_forward / residual_rms_forward
// (layernorm.py:16-33: x / sqrt(mean(x^2) + eps) * weight, after
// x = x + residual) and SiluAndMul (activation.py:16-19: silu(x[:, :I]) *
// x[:, I:]).  Each runs as several torch elementwise and reduction kernels in
// an eager model (about 9 launches per norm); here each is one HBM pass,
// which matters most in a decode step, where every launch covers only a few
// dozen rows.  Arithmetic is fp32 with one rounding to the element dtype at
// the end (the residual sum is rounded to the dtype first, as the residual
// stream is kept in that dtype).
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kRowWaves = 4;

// 8 consecutive elements of dtype DT as fp32 from one 16-byte (16-bit
// dtypes) or two 16-byte (fp32) loads.
template <int DT>
MKV_DEV void load8(const void* base, int64_t elem, float* x) {
  if constexpr (DT == MKV_DTYPE_F32) {
    const float* p = reinterpret_cast<const float*>(base) + elem;
    const u32x4 a = ld16(p), b = ld16(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = __uint_as_float(a[j]);
      x[4 + j] = __uint_as_float(b[j]);
    }
  } else {
    const u32x4 a = ld16(reinterpret_cast<const uint16_t*>(base) + elem);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = DT == MKV_DTYPE_BF16 ? bf16_bits_to_f32(a[j] & 0xffffu) : f16_bits_to_f32(a[j] & 0xffffu);
      x[2 * j + 1] = DT == MKV_DTYPE_BF16 ? bf16_bits_to_f32(a[j] >> 16) : f16_bits_to_f32(a[j] >> 16);
    }
  }
}

template <int DT>
MKV_DEV float round_to(float x) {
  if constexpr (DT == MKV_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  if constexpr (DT == MKV_DTYPE_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  return x;
}

template <int DT>
MKV_DEV void store8(void* base, int64_t elem, const float* x) {
  if constexpr (DT == MKV_DTYPE_F32) {
    float* p = reinterpret_cast<float*>(base) + elem;
    u32x4 a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = __float_as_uint(x[j]);
      b[j] = __float_as_uint(x[4 + j]);
    }
    st16(p, a);
    st16(p + 4, b);
  } else {
    u32x4 a;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = DT == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x[2 * j]) : f32_to_f16_bits(x[2 * j]);
      const uint32_t hi = DT == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
      a[j] = lo | (hi << 16);
    }
    st16(reinterpret_cast<uint16_t*>(base) + elem, a);
  }
}

// One wavefront per row; the row (up to kMaxChunks x 8 elements per lane)
// stays in registers between the sum of squares and the scaling.
constexpr int kMaxChunks = 4;  // hidden <= 64 * 8 * 4 = 2048 per pass of registers

template <int DT>
__global__ __launch_bounds__(kRowWaves* kWave) void rmsnorm_kernel(
    void* __restrict__ out, void* __restrict__ residual, const void* __restrict__ x,
    const void* __restrict__ weight, int64_t rows, int hidden, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * hidden;
  const int chunks = hidden / 8;
  float h[kMaxChunks][8], w[kMaxChunks][8];
  float ss = 0.0f;
  // the weight is loaded with the row (one memory round trip, not two)
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u)
    if (lane + 64 * u < chunks) load8<DT>(weight, 8 * (lane + 64 * u), w[u]);
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    const int c = lane + 64 * u;
    if (c < chunks) {
      load8<DT>(x, base + 8 * c, h[u]);
      if (residual) {
        float r[8];
        load8<DT>(residual, base + 8 * c, r);
#pragma unroll
        for (int j = 0; j < 8; ++j) h[u][j] = round_to<DT>(h[u][j] + r[j]);
        store8<DT>(residual, base + 8 * c, h[u]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(h[u][j], h[u][j], ss);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    const int c = lane + 64 * u;
    if (c < chunks) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = h[u][j] * inv * w[u][j];
      store8<DT>(out, base + 8 * c, y);
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(void* __restrict__ out,
                                                       const void* __restrict__ x, int64_t rows,
                                                       int inter, int64_t x_row_stride) {
  const int chunks = inter / 8;
  const int64_t total = rows * chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / chunks;
    const int c = (int)(i - r * chunks);
    float a[8], b[8], y[8];
    load8<DT>(x, r * x_row_stride + 8 * c, a);
    load8<DT>(x, r * x_row_stride + inter + 8 * c, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = a[j] / (1.0f + __expf(-a[j])) * b[j];
    store8<DT>(out, r * (int64_t)inter + 8 * c, y);
  }
}

int dtype_ok(int dt) { return dt == MKV_DTYPE_F32 || dt == MKV_DTYPE_BF16 || dt == MKV_DTYPE_F16; }

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_rmsnorm(void* out, void* residual, const void* x, const void* weight,
                           int64_t rows, int hidden, float eps, int dtype, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 64 * 8 * kMaxChunks) return MKV_ERR_BAD_SHAPE;
  if (!dtype_ok(dtype)) return MKV_ERR_UNSUPPORTED_DTYPE;
  if (rows == 0) return MKV_OK;
  if (!out || !x || !weight) return MKV_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual) |
       reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15u)
    return MKV_ERR_MISALIGNED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + kRowWaves - 1) / kRowWaves)), block(kRowWaves * kWave);
  switch (dtype) {
    case MKV_DTYPE_BF16:
      hipLaunchKernelGGL(rmsnorm_kernel<MKV_DTYPE_BF16>, grid, block, 0, s, out, residual, x, weight, rows, hidden, eps);
      break;
    case MKV_DTYPE_F16:
      hipLaunchKernelGGL(rmsnorm_kernel<MKV_DTYPE_F16>, grid, block, 0, s, out, residual, x, weight, rows, hidden, eps);
      break;
    default:
      hipLaunchKernelGGL(rmsnorm_kernel<MKV_DTYPE_F32>, grid, block, 0, s, out, residual, x, weight, rows, hidden, eps);
      break;
  }
  return (int)hipGetLastError();
}

extern "C" int mkv_silu_mul(void* out, const void* x, int64_t x_row_stride, int64_t rows,
                            int inter, int dtype, void* stream) {
  if (rows < 0 || inter <= 0 || inter % 8 || x_row_stride < 2 * (int64_t)inter) return MKV_ERR_BAD_SHAPE;
  if (!dtype_ok(dtype)) return MKV_ERR_UNSUPPORTED_DTYPE;
  if (rows == 0) return MKV_OK;
  if (!out || !x) return MKV_ERR_NULL_POINTER;
  const int eb = dtype == MKV_DTYPE_F32 ? 4 : 2;
  if (((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(x)) & 15u) || (x_row_stride * eb) % 16)
    return MKV_ERR_MISALIGNED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = rows * (inter / 8);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  switch (dtype) {
    case MKV_DTYPE_BF16:
      hipLaunchKernelGGL(silu_mul_kernel<MKV_DTYPE_BF16>, dim3((unsigned)blocks), dim3(256), 0, s, out, x, rows, inter, x_row_stride);
      break;
    case MKV_DTYPE_F16:
      hipLaunchKernelGGL(silu_mul_kernel<MKV_DTYPE_F16>, dim3((unsigned)blocks), dim3(256), 0, s, out, x, rows, inter, x_row_stride);
      break;
    default:
      hipLaunchKernelGGL(silu_mul_kernel<MKV_DTYPE_F32>, dim3((unsigned)blocks), dim3(256), 0, s, out, x, rows, inter, x_row_stride);
      break;
  }
  return (int)hipGetLastError();
}
