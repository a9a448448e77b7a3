// Decode-step metadata on the device.
//
// Reference: ModelRunner.prepare_decode (model_runner.py:621-640) builds, on
// the host and for every decode step, context_lens[b] = len(seq) and
// slot_mapping[b] = block_table[-1] * block_size + last_block_num_tokens - 1
// (the slot of the token being decoded), then copies both to the device;
// run_model (:681-706) copies them again into the captured graph's buffers.
// Here the runner keeps per-row sequence lengths and block tables resident on
// the device and one small kernel derives the step's metadata from them, so a
// decode step needs no host lists and no host-to-device copy (the host only
// writes a block-table entry when a sequence gets a new block, and a row when
// a sequence joins), and the kernel itself can sit inside a captured graph.
#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kMetaThreads = 256;

// Row b of `rows`: an active row (seq_lens[b] > 0) advances by `increment`
// tokens; its context length is the new length L and the slot of token L - 1
// is block_tables[b, (L-1) / bs] * bs + (L-1) % bs, or -1 when that entry is
// absent (-1 or outside the pool).  Inactive rows (seq_lens[b] <= 0, e.g. the
// padding rows of a captured batch) get context length 0 and slot -1, which
// the append skips and the decode writes as zeros.
__global__ __launch_bounds__(kMetaThreads) void decode_metadata_kernel(
    int64_t* __restrict__ seq_lens, int64_t* context_lens, int64_t* __restrict__ slot_mapping,
    const int32_t* __restrict__ block_tables, int64_t bt_stride, int max_blocks,
    int64_t num_blocks, int bs_log2, int rows, int increment) {
  const int b = blockIdx.x * kMetaThreads + threadIdx.x;
  if (b >= rows) return;
  int64_t L = seq_lens[b];
  int64_t slot = -1;
  if (L > 0) {
    L += increment;
    const int64_t t = L - 1;
    const int64_t blk = t >> bs_log2;
    if (blk < max_blocks) {
      const int64_t p = block_tables[(int64_t)b * bt_stride + blk];
      if (p >= 0 && p < num_blocks) slot = (p << bs_log2) + (t & ((int64_t(1) << bs_log2) - 1));
    }
  } else {
    L = 0;
  }
  seq_lens[b] = L;
  context_lens[b] = L;
  slot_mapping[b] = slot;
}

int ilog2_pow2(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_decode_metadata(int64_t* seq_lens, int64_t* context_lens, int64_t* slot_mapping,
                                   const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                   int64_t num_blocks, int block_size, int rows, int increment,
                                   void* stream) {
  if (rows < 0 || max_blocks < 0 || num_blocks < 0 || increment < 0) return MKV_ERR_BAD_SHAPE;
  if (rows == 0) return MKV_OK;
  if (!seq_lens || !context_lens || !slot_mapping || (max_blocks > 0 && !block_tables))
    return MKV_ERR_NULL_POINTER;
  if (bt_stride < max_blocks) return MKV_ERR_BAD_STRIDE;
  const int bs_log2 = ilog2_pow2(block_size);
  if (bs_log2 < 0) return MKV_ERR_BAD_BLOCK_SIZE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(decode_metadata_kernel, dim3((unsigned)((rows + kMetaThreads - 1) / kMetaThreads)),
                     dim3(kMetaThreads), 0, s, seq_lens, context_lens, slot_mapping, block_tables,
                     bt_stride, max_blocks, num_blocks, bs_log2, rows, increment);
  return (int)hipGetLastError();
}
