// K4 (standalone form): paged -> contiguous gather through the block table.
//
// Reference: the torch gather of benchmark_decoding.py:166-178 and the inline
// address arithmetic of every paged kernel (attention.py:578-590, :787-798).
// One wavefront copies one token row (all KV heads) with 16-byte accesses;
// rows past context_lens[b] or in an absent block (-1) are zero-filled.
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kGatherWaves = 4;

__global__ __launch_bounds__(kGatherWaves* kWave) void gather_kv_kernel(
    char* __restrict__ dst, const char* __restrict__ cache, PagedIndex idx,
    const void* __restrict__ context_lens, int ctx_i64, int batch, int64_t max_len,
    int elem_bytes) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kGatherWaves + (threadIdx.x >> 6);
  if (row >= (int64_t)batch * max_len) return;
  const int b = (int)(row / max_len);
  const int64_t t = row - (int64_t)b * max_len;
  const int64_t L = load_index(context_lens, b, ctx_i64);
  const int64_t phys = t < L ? idx.physical_block(b, t >> idx.bs_log2) : -1;
  const int64_t row_bytes = idx.row_elems * elem_bytes;
  char* d = dst + row * row_bytes;
  if (phys < 0) {
    for (int64_t o = (int64_t)lane * 16; o < row_bytes; o += kWave * 16) st16(d + o, u32x4{0, 0, 0, 0});
    return;
  }
  const char* s = cache + idx.row_offset(phys, t) * elem_bytes;
  for (int64_t o = (int64_t)lane * 16; o < row_bytes; o += kWave * 16) st16(d + o, ld16(s + o));
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_gather_kv(void* dst, const void* cache, int dtype, int64_t num_blocks,
                             const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                             const void* context_lens, int context_lens_dtype, int batch,
                             int max_len, int num_kv_heads, int head_dim, int block_size,
                             void* stream) {
  if (batch < 0 || max_len < 0 || num_kv_heads <= 0 || head_dim <= 0 || max_blocks < 0 ||
      num_blocks < 0)
    return MKV_ERR_BAD_SHAPE;
  if (batch == 0 || max_len == 0) return MKV_OK;
  if (!dst || !cache || !block_tables || !context_lens) return MKV_ERR_NULL_POINTER;
  int eb;
  switch (dtype) {
    case MKV_DTYPE_F32: eb = 4; break;
    case MKV_DTYPE_BF16:
    case MKV_DTYPE_F16: eb = 2; break;
    case MKV_DTYPE_FP8E4M3:
    case MKV_DTYPE_I8: eb = 1; break;
    default: return MKV_ERR_UNSUPPORTED_DTYPE;
  }
  if (context_lens_dtype != MKV_INDEX_I32 && context_lens_dtype != MKV_INDEX_I64)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 0) return MKV_ERR_BAD_BLOCK_SIZE;
  if (bt_stride < max_blocks) return MKV_ERR_BAD_STRIDE;
  const int64_t row_bytes = (int64_t)num_kv_heads * head_dim * eb;
  if (row_bytes % 16) return MKV_ERR_BAD_SHAPE;
  if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(cache)) & 15u)
    return MKV_ERR_MISALIGNED;
  PagedIndex idx;
  idx.block_tables = block_tables;
  idx.bt_stride = bt_stride;
  idx.max_blocks = max_blocks;
  idx.num_blocks = num_blocks;
  idx.bs_log2 = bs_log2;
  idx.row_elems = (int64_t)num_kv_heads * head_dim;
  const int64_t rows = (int64_t)batch * max_len;
  hipLaunchKernelGGL(gather_kv_kernel, dim3((unsigned)((rows + kGatherWaves - 1) / kGatherWaves)),
                     dim3(kGatherWaves * kWave), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<char*>(dst), reinterpret_cast<const char*>(cache), idx,
                     context_lens, (int)(context_lens_dtype == MKV_INDEX_I64), batch,
                     (int64_t)max_len, eb);
  return (int)hipGetLastError();
}
