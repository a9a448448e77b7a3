// ABI version and status strings of libmkv (host-only code).
#include <hip/hip_runtime.h>

#include "mkv.h"

extern "C" int mkv_abi_version(void) { return MKV_ABI_VERSION; }

extern "C" const char* mkv_status_string(int status) {
  switch (status) {
    case MKV_OK: return "ok";
    case MKV_ERR_NULL_POINTER: return "a required pointer argument is NULL";
    case MKV_ERR_BAD_SHAPE: return "invalid shape or size argument";
    case MKV_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype combination";
    case MKV_ERR_UNSUPPORTED_HEAD_DIM:
      return "unsupported head_dim (attention kernels: 128; per-token-head append: a power of two in 16..1024)";
    case MKV_ERR_UNSUPPORTED_GROUP:
      return "num_heads must be a multiple of num_kv_heads with a group size in 1..16";
    case MKV_ERR_BAD_BLOCK_SIZE: return "block_size must be a power of two (>= 16 for attention)";
    case MKV_ERR_WORKSPACE_TOO_SMALL: return "workspace is smaller than the size query reported";
    case MKV_ERR_MISALIGNED: return "pointer or row stride is not 16-byte aligned";
    case MKV_ERR_BAD_STRIDE: return "row stride is smaller than the row it must hold";
    case MKV_ERR_SCRATCH_LIMIT:
      return "the call needs more than the library's static per-device scratch "
             "(MKV_NOALLOC_SCRATCH_BYTES); use mkv_paged_decode with a workspace";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown mkv status";
}
