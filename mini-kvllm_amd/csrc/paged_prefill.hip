// K3: causal prefill / extend attention on the MFMA units, over the paged
// KV cache (chunked prefill) or over fresh contiguous K/V (full prefill).
//
// Reference semantics: paged_attention_prefill_kernel (attention.py:704-847,
// wrapper :852-891; visible = min(context_len, position + 1) at :747) and
// flash_attention_varlen_kernel (attention.py:336-443, wrapper :446-514).
// FP8 caches are dequantised exactly (e4m3fn -> fp16) as their tiles are
// staged into LDS, which the reference leaves unimplemented
// (attention.py:1702-1708).
//
// Work decomposition: a workgroup of 8 wavefronts owns 128 "rows" of one
// sequence and one KV head, where a row is a (query token, query head of the
// GQA group) pair, token-major; every row of the group reads the same K/V,
// so each K/V tile is staged in LDS once for G query heads.  Tiles of 64 keys
// are gathered through the block table into double-buffered LDS with an XOR
// swizzle on 16-byte chunks (every LDS access conflict-free): 16-bit caches
// by LDS DMA (buffer_load ... lds), FP8 / INT8 caches through registers,
// converted on the way.  Each wave
// owns one row tile of 16 and computes
//   S^T = K Q^T     (A = K from LDS, B = Q^T resident in registers)
//   O  += P V       (A = P straight from the S^T accumulators, B = V read
//                    from LDS already transposed by ds_read_b64_tr_b16)
// with an online softmax in the log2 domain whose output rescale is deferred
// until a row's running max grows by more than 2^8.  The varlen tile list
// (longest sequences first, each sequence's last tile first) is built on the
// device — by every workgroup in LDS for up to 256 sequences, else by a
// one-workgroup scan kernel — so the launch needs no host sync; with a
// multiple of 8 KV heads the grid is ordered so that all tiles of one KV head
// run on one XCD and share its L2.
#include <type_traits>

#include "mkv_device.hpp"

namespace mkv {
namespace {

constexpr int kHeadDim = 128;
constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kRowTiles = 1;                       // 16-row MFMA tiles per wave
constexpr int kRowsPerWg = kPfWaves * kRowTiles * 16;  // 128
static_assert(kRowsPerWg == 2 * kWave, "the row visibility reduction assumes the rows fill waves 0 and 1");
constexpr int kBN = 64;                            // keys per LDS tile
// static LDS: 4 tiles of 64 keys x 256 bytes (K and V, double-buffered);
// dynamic LDS: row visibility [128] + 4 ints, per-token scales [2][256]
// (per tile buffer: K then V scales of the tile's 64 keys, and with head
// pairing the same for the pair's second KV head), the largest V scale of
// each buffer's tile [2][2] (per KV head of a pair), then the inline tile
// list (8-aligned)
constexpr int kScPerBuf = 256;
constexpr int kTileListOffset = (128 + 4) * 4 + 2 * kScPerBuf * 4 + 4 * 4;
static_assert(kTileListOffset % 8 == 0, "TilePick holds 64-bit fields");
constexpr int kXcds = 8;
constexpr float kNegBig = -1e30f;
constexpr float kRescaleSlack = 8.0f;
// bf16 P·V operands: bf16 holds P to 8 bits, so P (fp32) is split into bf16
// hi + lo terms (~16-bit P, two MFMAs per step) on every key.  One term (the
// reference's flash kernel rounds P once, p.to(v.dtype), attention.py:432)
// misses 2e-3 where a row's weight sits on two or three keys: the error is
// ~2^-9 * w_i w_j |v_i - v_j|.  fp16 operands (FP8 caches) take one term, an
// 11-bit P.

struct PrefillArgs {
  void* out;
  const void* q;
  int q_dtype;
  const char* k;  // paged pool (N, bs, Hkv, D) or contiguous (total, Hkv, D)
  const char* v;
  const float* k_scale;
  const float* v_scale;
  PagedIndex idx;  // paged only
  const void* context_lens;
  int ctx_i64;
  const int32_t* cu_seqlens_q;
  const int64_t* positions;  // paged only
  int num_seqs;
  int64_t total_q;
  int num_heads;
  int num_kv_heads;
  int group;
  int tok_per_wg;
  float sm_scale;
  int32_t* tile_start;  // [num_seqs + 1], over the visiting order
  const int32_t* order; // [num_seqs]: sequence visited at position k
  int inline_list;      // num_seqs <= kInlineSeqs: each workgroup builds the list in LDS
  int64_t tiles_ub;     // upper bound of tiles per KV head (grid rows)
  int scale_heads;      // KV heads of the per-token-head scale tensors (the caller's Hkv)
  int pair;             // head_dim 64: KV heads read in pairs (kQDim in mkv_device.hpp)
};

// ---------------------------------------------------------------------------
// Tile list.  Sequences are visited longest first (by context length, paged;
// by query length, contiguous), and each sequence's tiles from its last (the
// rows that see the most keys) to its first: the grid then hands out the
// workgroups roughly longest-processing-time first, which keeps the last
// workgroups of a launch short.  order[k] = the sequence at position k,
// tile_start[k] = sum_{k' < k} ceil(qlen(order[k']) / tok_per_wg).  Batches
// of more than 256 sequences keep their own order.  The order changes which
// workgroup computes a tile, never the tile's result.
// ---------------------------------------------------------------------------
// Up to kInlineSeqs sequences: every prefill workgroup finds its own tile
// (pick_tile_inline: no scan launch, no global lookups of the tile's
// sequence); the scan kernel builds the list in LDS when a caller asks for
// the global list.
constexpr int kInlineSeqs = 256;
struct TileListLds {
  int32_t part[kInlineSeqs];
  int32_t key[kInlineSeqs];
  int32_t ord[kInlineSeqs];
  int32_t ts[kInlineSeqs + 1];   // tile prefix over the visiting order
  int32_t cu[kInlineSeqs + 1];   // cu_seqlens_q
  int32_t ctx[kInlineSeqs];      // clamped context lengths (paged)
};

// Builds the list of n <= kInlineSeqs sequences in L with one coalesced
// round trip for cu_seqlens_q and context_lens; the first kInlineSeqs
// threads do the per-sequence work, and every thread of the workgroup must
// call it (it holds barriers).
MKV_DEV void build_tile_list(TileListLds& L, const int32_t* __restrict__ cu, const void* context_lens,
                             int ctx_i64, int64_t ctx_cap, int n, int tok_per_wg) {
  const int t = threadIdx.x;
  if (t <= n) L.cu[t] = cu[t];
  if (t < n) {
    int64_t c = context_lens ? load_index(context_lens, t, ctx_i64) : 0;
    c = c < 0 ? 0 : (c > ctx_cap ? ctx_cap : c);
    L.ctx[t] = (int32_t)(c < 0x7fffffff ? c : 0x7fffffff);
  }
  __syncthreads();
  int32_t kk = -1;
  if (t < n) {
    const int32_t len = L.cu[t + 1] - L.cu[t];
    if (len > 0) kk = context_lens ? L.ctx[t] : len;
    L.key[t] = kk;
  }
  __syncthreads();
  if (t < n) {  // stable rank, longest first
    int r = 0;
    for (int j = 0; j < n; ++j) {
      const int32_t kj = L.key[j];
      r += (kj > kk) || (kj == kk && j < t);
    }
    L.ord[r] = t;
  }
  __syncthreads();
  const int s = t < n ? L.ord[t] : 0;
  const int32_t len = t < n ? L.cu[s + 1] - L.cu[s] : 0;
  const int32_t nt = len > 0 ? (len + tok_per_wg - 1) / tok_per_wg : 0;
  // Inclusive scan of nt over the kInlineSeqs entries: each of the first
  // kInlineSeqs / 64 waves scans its 64 entries with lane shuffles, then adds
  // the totals of the waves before it (one barrier, where a workgroup-wide
  // Hillis-Steele scan takes two per step).
  const int lane = t & 63;
  int32_t incl = nt;
  if (t < kInlineSeqs) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    if (lane == 63) L.part[t >> 6] = incl;
  }
  __syncthreads();
  int32_t total = 0;
#pragma unroll
  for (int w = 0; w < kInlineSeqs / 64; ++w) {
    const int32_t p = L.part[w];
    if (w < (t >> 6)) incl += p;
    total += p;
  }
  if (t < n) L.ts[t] = incl - nt;
  if (t == 0) L.ts[n] = total;
  __syncthreads();
}

// The tile `tau` of the longest-first list of n <= kInlineSeqs sequences,
// found without building the list: a sequence's first tile in that order is
// the sum of the tile counts of the sequences before it (longer key first,
// ties in batch order), which one pass over the n sequences gives.  Waves
// w < ceil(n / 64) own sequences 64w + lane: each lane writes its sequence's
// order value and tile count to LDS once, then reads all n entries with
// uniform-address reads (LDS broadcasts, 8 entries per step, no scan, no
// search); the one lane whose sequence holds tile tau writes it out, and
// P.seq stays -1 when no sequence does.  ~1.7 us per workgroup less than
// the LDS list (a rank loop waiting on one LDS read per sequence, a scan
// and a binary search: ~3.9 us for 60 prompts).  Every thread of the
// workgroup must call it (one barrier; two for more than 64 sequences).
struct TilePick {
  int32_t seq;    // -1: no tile
  int32_t tile;   // the tile's index within its sequence's tiles
  int64_t q_seq0, q_seq1;
  int64_t ctx;    // clamped context length (paged)
  uint2 ent[kInlineSeqs];  // order value, tile count (0, 0 past n)
};
template <bool PAGED>
MKV_DEV void pick_tile_inline(const PrefillArgs& a, TilePick& P, int64_t tau, int64_t ctx_cap) {
  const int t = threadIdx.x;
  const int n = a.num_seqs;
  const int nw = (n + 63) >> 6;
  const bool active = t < 64 * nw;
  // Sequence t's order value: (key + 1) * 256 + 255 - t, with the key capped
  // at 2^23 - 2 (the cap only reorders sequences longer than 8M tokens among
  // themselves) and key -1 for an empty sequence; sequence j comes before
  // sequence t when its value is larger (longer key, or the same key and
  // j < t).  n <= 256 keeps t in the low byte.
  uint32_t ov = 0;
  int32_t nt = 0, c0 = 0, c1 = 0, cx = 0;
  if (active) {
    if (t < n) {
      c0 = a.cu_seqlens_q[t];
      c1 = a.cu_seqlens_q[t + 1];
      if (PAGED && a.context_lens != nullptr) {
        int64_t c = load_index(a.context_lens, t, a.ctx_i64);
        c = c < 0 ? 0 : (c > ctx_cap ? ctx_cap : c);
        cx = (int32_t)(c < 0x7fffffff ? c : 0x7fffffff);
      }
      const int32_t len = c1 - c0;
      if (len > 0) {
        const int32_t key = (PAGED && a.context_lens != nullptr) ? cx : len;
        ov = ((uint32_t)(key < (1 << 23) - 2 ? key : (1 << 23) - 2) + 1u) << 8;
        nt = (len + a.tok_per_wg - 1) / a.tok_per_wg;
      }
      ov |= 255u - (uint32_t)t;
    }
    if (t == 0) P.seq = -1;
    P.ent[t] = make_uint2(ov, (uint32_t)nt);
  }
  // (one wave: its LDS writes complete before its reads, in order)
  if (nw > 1) __syncthreads();
  if (active) {
    int32_t ts = 0;
    for (int j0 = 0; j0 < n; j0 += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint2 e = P.ent[j0 + u];
        ts += e.x > ov ? (int32_t)e.y : 0;
      }
    }
    if (nt > 0 && (int64_t)ts <= tau && tau < (int64_t)ts + nt) {
      P.seq = t;
      P.tile = ts + nt - 1 - (int32_t)tau;  // the sequence's last tile first
      P.q_seq0 = c0;
      P.q_seq1 = c1;
      P.ctx = cx;
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Tile list kernel (batches of more than kInlineSeqs sequences, in batch
// order; smaller ones only when a caller asks for the global list).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_tile_scan_kernel(const int32_t* __restrict__ cu,
                                                                const void* context_lens, int ctx_i64,
                                                                int64_t ctx_cap, int num_seqs,
                                                                int tok_per_wg,
                                                                int32_t* __restrict__ tile_start,
                                                                int32_t* __restrict__ order) {
  __shared__ TileListLds L;
  const int t = threadIdx.x;
  if (num_seqs <= kInlineSeqs) {
    build_tile_list(L, cu, context_lens, ctx_i64, ctx_cap, num_seqs, tok_per_wg);
    if (t < num_seqs) {
      tile_start[t] = L.ts[t];
      order[t] = L.ord[t];
    }
    if (t == 0) tile_start[num_seqs] = L.ts[num_seqs];
    return;
  }
  int32_t running = 0;
  for (int base = 0; base < num_seqs; base += 256) {
    const int s = base + t;
    int32_t n = 0;
    if (s < num_seqs) {
      const int32_t len = cu[s + 1] - cu[s];
      n = len > 0 ? (len + tok_per_wg - 1) / tok_per_wg : 0;
    }
    L.part[t] = n;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // Hillis-Steele inclusive scan
      const int32_t add = t >= off ? L.part[t - off] : 0;
      __syncthreads();
      L.part[t] += add;
      __syncthreads();
    }
    if (s < num_seqs) {
      tile_start[s] = running + L.part[t] - n;
      order[s] = s;
    }
    running += L.part[255];
    __syncthreads();
  }
  if (t == 0) tile_start[num_seqs] = running;
}

template <int KV_DT>
using Op16 = typename std::conditional<KV_DT == MKV_DTYPE_BF16, bf16x8, f16x8>::type;

template <int KV_DT>
MKV_DEV f32x4 mfma16(Op16<KV_DT> A, Op16<KV_DT> B, f32x4 C) {
  if constexpr (KV_DT == MKV_DTYPE_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, C, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, C, 0, 0, 0);
}

template <int KV_DT>
MKV_DEV Op16<KV_DT> to_op16(const float* x) {
  Op16<KV_DT> r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (KV_DT == MKV_DTYPE_BF16)
      r[j] = (__bf16)x[j];
    else
      r[j] = (_Float16)x[j];
  }
  return r;
}

MKV_DEV void store_out8(void* out, int dt, int64_t off, const float* x) {
  if (dt == MKV_DTYPE_F32) {
    float* p = reinterpret_cast<float*>(out) + off;
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
      const uint32_t lo = dt == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x[2 * j]) : f32_to_f16_bits(x[2 * j]);
      const uint32_t hi = dt == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
      a[j] = lo | (hi << 16);
    }
    st16(reinterpret_cast<uint16_t*>(out) + off, a);
  }
}

// max(x, x of lane ^ 16) and max(x, x of lane ^ 32): VALU lane swaps
// (v_permlane16_swap / v_permlane32_swap) that leave each lane the pair of
// its own and its partner's value, with no LDS round trip or address
// register.
// The max is one v_max_f32: through fmaxf the compiler first quiets each
// swapped operand (v_max_f32 x, x, x) since it cannot see that they hold no
// signalling NaN; the scores, MFMA results and their maxima, never do.
MKV_DEV float vmax_quiet(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
MKV_DEV float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax_quiet(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
MKV_DEV float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax_quiet(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Maximum over the wave's 64 lanes by DPP moves (quad_perm xor 1 and xor 2,
// the half-row and row mirrors) and the two lane swaps: no lane index
// arithmetic (__shfl_xor's would stay live across the key loop) and no LDS.
MKV_DEV float wave_max_dpp(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xf, 0xf, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xf, 0xf, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xf, 0xf, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xf, 0xf, false)));
  return max_xor32(max_xor16(x));
}

// A workgroup-uniform 64-bit value in scalar registers.
MKV_DEV int64_t uniform_i64(int64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// mask bit of the lane set ? b : a, as one v_cndmask_b32 (opaque to LLVM,
// which folds two such selects of one vector into a dynamic index)
MKV_DEV uint32_t lane_select(uint32_t a, uint32_t b, uint64_t mask) {
  uint32_t r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
  return r;
}

// The lane index, computed where it is used: a volatile asm pair that the
// compiler can neither hoist out of a loop nor keep in a register across it.
MKV_DEV int lane_id_volatile() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// The workgroup's share of a prefill launch: its KV head, sequence and
// query rows, and the number of keys each of its kRowsPerWg rows sees.
struct WgWork {
  int kvh;
  int seq;
  int64_t q_seq0;  // first query row of the sequence
  int64_t q0, q1;  // the workgroup's query rows [q0, q1)
  int64_t ctx;     // keys of the sequence (paged: its clamped context length)
  int min_vis, max_vis;
};

// Looks up the workgroup's tile (XCD-aware order over the longest-first
// tile list).  Returns false, uniformly over the workgroup, when it has no
// tile.  Holds barriers: every thread of the workgroup must call it.
template <bool PAGED>
MKV_DEV bool wg_tile(const PrefillArgs& a, char* smem, WgWork& w) {
  // XCD-aware order: with a multiple of 8 KV heads every XCD takes whole
  // heads (consecutive logical tiles share an XCD and its L2, and each XCD
  // sees the same longest-first mix); otherwise the tiles are dealt round
  // robin, so that the longest ones spread over all XCDs.
  const int64_t nwg = gridDim.x;
  const int64_t logical = a.num_kv_heads % kXcds == 0
                              ? (int64_t)(blockIdx.x % kXcds) * (nwg / kXcds) + blockIdx.x / kXcds
                              : (int64_t)blockIdx.x;
  const int kvh = (int)(logical / a.tiles_ub);
  const int64_t tau = logical - (int64_t)kvh * a.tiles_ub;
  if (kvh >= a.num_kv_heads) return false;
  const int64_t cap = PAGED ? (int64_t)a.idx.max_blocks << a.idx.bs_log2 : 0;
  int seq;
  int64_t q_seq0, q_seq1, tile, ctx;
  if (a.inline_list) {
    TilePick& P = *reinterpret_cast<TilePick*>(smem + kTileListOffset);
    pick_tile_inline<PAGED>(a, P, tau, cap);
    if (P.seq < 0) return false;
    seq = P.seq;
    q_seq0 = P.q_seq0;
    q_seq1 = P.q_seq1;
    tile = P.tile;
    ctx = PAGED ? P.ctx : q_seq1 - q_seq0;
  } else {
    if (tau >= a.tile_start[a.num_seqs]) return false;
    int lo = 0, hi = a.num_seqs;  // largest k with tile_start[k] <= tau
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.tile_start[mid] <= tau) lo = mid; else hi = mid;
    }
    seq = a.order[lo];
    q_seq0 = a.cu_seqlens_q[seq];
    q_seq1 = a.cu_seqlens_q[seq + 1];
    tile = (int64_t)(a.tile_start[lo + 1] - 1) - tau;  // the sequence's last tile first
    if constexpr (PAGED) {
      ctx = load_index(a.context_lens, seq, a.ctx_i64);
      ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
    } else {
      ctx = q_seq1 - q_seq0;
    }
  }
  // The sequence's rows are clamped to [0, total_q): a cu_seqlens_q whose
  // entries leave that range (the kernel cannot check them on the host
  // without a sync) loses those rows instead of reading or writing past q
  // and out.
  q_seq0 = q_seq0 < 0 ? 0 : (q_seq0 > a.total_q ? a.total_q : q_seq0);
  q_seq1 = q_seq1 < q_seq0 ? q_seq0 : (q_seq1 > a.total_q ? a.total_q : q_seq1);
  if constexpr (!PAGED) ctx = q_seq1 - q_seq0;
  w.kvh = kvh;
  w.seq = seq;
  w.q_seq0 = q_seq0;
  w.q0 = q_seq0 + tile * (int64_t)a.tok_per_wg;
  w.q1 = w.q0 + a.tok_per_wg < q_seq1 ? w.q0 + a.tok_per_wg : q_seq1;
  w.ctx = ctx;
  return true;
}

// Keys seen by row `row` of a workgroup over contiguous K/V (0 for padding
// rows): visible = min(ctx, position + 1), the position counted from the
// sequence's first query token.
MKV_DEV int row_vis_contiguous(const PrefillArgs& a, const WgWork& w, int row) {
  const int64_t tok = w.q0 + row / a.group;
  if (row >= a.tok_per_wg * a.group || tok >= w.q1) return 0;
  const int64_t v = tok - w.q_seq0 + 1;
  return (int)(v < w.ctx ? v : w.ctx);
}

// The number of keys each of the workgroup's kRowsPerWg rows sees, in
// vis_lds[row] (0 for padding rows; paged), and their min / max over the real
// rows.  Holds a barrier when paged: every thread of the workgroup must call
// it.
template <bool PAGED>
MKV_DEV void wg_rows(const PrefillArgs& a, int* vis_lds, int* red_lds, WgWork& w) {
  if constexpr (!PAGED) {
    // contiguous K/V: a row's visibility grows with its token, so the real
    // rows' min / max are those of the first and the last token, and each
    // row's own comes from row_vis_contiguous (no LDS, no barrier)
    w.min_vis = (int)(w.q0 - w.q_seq0 + 1 < w.ctx ? w.q0 - w.q_seq0 + 1 : w.ctx);
    w.max_vis = (int)(w.q1 - w.q_seq0 < w.ctx ? w.q1 - w.q_seq0 : w.ctx);
    return;
  }
  const int tid = threadIdx.x;
  const int64_t q0 = w.q0, q1 = w.q1, q_seq0 = w.q_seq0, ctx = w.ctx;
  const int G = a.group;
  if (tid < kRowsPerWg) {
    const int64_t tok = q0 + tid / G;
    int vis = 0;
    if (tid < a.tok_per_wg * G && tok < q1) {
      const int64_t pos = PAGED ? a.positions[tok] : tok - q_seq0;
      const int64_t v = pos + 1 < ctx ? pos + 1 : ctx;
      vis = v < 0 ? 0 : (int)v;
    }
    vis_lds[tid] = vis;
    // min / max over the real rows: the rows are waves 0 and 1; each reduces
    // its 64 with lane shuffles and writes one pair (LDS atomics from every
    // row to one address serialise: ~7 us per workgroup)
    const bool real = tid < a.tok_per_wg * G && tok < q1;
    int mn = real ? vis : 0x7fffffff, mx = real ? vis : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      mn = min(mn, __shfl_xor(mn, off));
      mx = max(mx, __shfl_xor(mx, off));
    }
    if ((tid & 63) == 0) {
      red_lds[2 * (tid >> 6)] = mn;
      red_lds[2 * (tid >> 6) + 1] = mx;
    }
  }
  __syncthreads();
  w.min_vis = min(red_lds[0], red_lds[2]);
  w.max_vis = max(red_lds[1], red_lds[3]);
}

// LDS geometry of one K or V tile: kBN key rows of 256 bytes (128 16-bit
// elements; FP8 caches are converted to fp16 as they are staged), 16-byte
// chunks XOR-swizzled by the key index.  The LDS serves 256 bytes per clock
// from 64 four-byte banks: 16 lanes of a 16-byte access, or 32 lanes of an
// 8-byte one, go together, and they are conflict-free when they touch 16
// distinct 16-byte positions of a 256-byte row (a row's chunk index).
// s(key) = ((key & 7) << 1) | ((key >> 3) & 1) is a bijection on key mod 16
// (K operand reads: 16 lanes, keys 16kt + c, one chunk) whose upper 3 bits
// are a bijection on 8 consecutive keys (V transposed reads: 32 lanes, keys
// 4kg + i, chunk pairs 2mm, 2mm + 1).  A 16-bit cache's LDS DMA writes whole
// 256-byte rows (the swizzle is applied to the global addresses instead); an
// FP8 / INT8 cache's staging writes go 8 lanes at a time over 32 banks, and
// its chunk pairs are split so that each write touches 8 distinct positions
// mod 8.  The V
// read offsets are computed for the first keys and reused 16 and 32 rows
// further, the staging offsets 16-48 rows further: s has period 16.
template <int KV_DT>
struct LdsTile {
  static constexpr int kEb = 2;
  static constexpr int kRowBytes = kHeadDim * kEb;  // 256
  static constexpr int kChunks = kRowBytes / 16;    // 16
  static constexpr int kBytes = kBN * kRowBytes;
  MKV_DEV static int swz(int key) { return ((key & 7) << 1) | ((key >> 3) & 1); }
  MKV_DEV static int offset(int key, int chunk) { return key * kRowBytes + ((chunk ^ swz(key)) << 4); }
};

// Four waves per SIMD (two 8-wave workgroups per CU) hide the latency of each
// wave's QK -> softmax -> PV chain, which leaves MFMA, VALU and LDS all far
// from busy at two waves per SIMD; the compiler keeps the kernel within 128
// registers, and the paged variants hold nothing in scratch inside the key
// loop (a reload there waits for the tile prefetch as well).
// QSPLIT (bf16 caches with an fp32 / fp16 q, per-token-head caches with an
// fp32 q): the operand type holds such a q to 8 (bf16) or 11 (fp16) bits, so
// q is split into hi + lo terms and each QK step takes a second MFMA, giving
// ~16 or more significant bits like the fp32 reference.
template <int KV_DT, bool PAGED, bool QSPLIT, bool PAIR>
MKV_DEV void prefill_mfma_body(const PrefillArgs& a) {
  using LT = LdsTile<KV_DT>;
  // CT: the element type of the LDS tiles and the MFMA operands (fp16 for
  // 1-byte caches, converted exactly while staging).
  // Per-token-head FP8 / INT8 caches: codes staged as exact fp16, scales
  // applied per key (K scale to the score, V scale to P, which stays one
  // fp16 term: the running max is raised where a tile's V scales would take
  // P * v_scale past the fp16 range, see the softmax below).
  constexpr bool kTokScale = kPerTokenScale<KV_DT>;
  constexpr int CT = (KV_DT == MKV_DTYPE_FP8E4M3 || kTokScale) ? MKV_DTYPE_F16 : KV_DT;
  constexpr int kEbG = DTypeInfo<KV_DT>::kBytes;  // cache element bytes
  constexpr int kChunksG = kHeadDim * kEbG / 16;   // 16-byte chunks per cache row
  extern __shared__ __align__(16) char smem[];
  // 16-bit caches stage tiles by LDS DMA into four distinct static buffers,
  // indexed by compile-time constants (below): the compiler's wait-count pass
  // then tells a read of one buffer from a pending DMA into the other and
  // lets the DMA run on under the reads.  Converting formats index one array
  // (buffer b: K at 2b tiles, V after it).
  constexpr bool kDma = DTypeInfo<KV_DT>::kBytes == 2;
  constexpr int kSplitBytes = kDma ? LT::kBytes : 16, kOneBytes = kDma ? 16 : 4 * LT::kBytes;
  __shared__ __align__(16) char lds_k0[kSplitBytes], lds_v0[kSplitBytes], lds_k1[kSplitBytes], lds_v1[kSplitBytes];
  __shared__ __align__(16) char lds_kv[kOneBytes];
#define KBUF(b) (kDma ? ((b) ? lds_k1 : lds_k0) : lds_kv + (b) * 2 * LT::kBytes)
#define VBUF(b) (kDma ? ((b) ? lds_v1 : lds_v0) : lds_kv + (b) * 2 * LT::kBytes + LT::kBytes)
  int* vis_lds = reinterpret_cast<int*>(smem);  // [kRowsPerWg]
  int* red_lds = vis_lds + kRowsPerWg;                             // [2]
  // per-token-head scales of the staged tiles: [buffer][K keys 0..63, V keys 0..63]
  float* sc_lds = reinterpret_cast<float*>(red_lds + 4);
  float* vmax_lds = sc_lds + 2 * kScPerBuf;  // [buffer][KV head of a pair]: the tile's largest V scale
  static_assert(kTileListOffset == (kRowsPerWg + 4) * 4 + 2 * kScPerBuf * 4 + 4 * 4, "LDS layout");

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, kg = lane >> 4;

  // The prologue (tile list, q, row visibility, first tile) and the epilogue
  // are chains of memory round trips that need few issue slots: they run at
  // the highest wave priority, so that the MFMA phases of the other
  // workgroup on the CU (raised to 1 below) do not hold them back.
  __builtin_amdgcn_s_setprio(3);
  WgWork wk;
  if (!wg_tile<PAGED>(a, smem, wk)) return;
  const int kvh = wk.kvh, seq = wk.seq;
  // (uniform: in scalar registers, not held in vector registers across the
  // key loop for the epilogue)
  const int64_t q_seq0 = uniform_i64(wk.q_seq0), q0 = uniform_i64(wk.q0), q1 = uniform_i64(wk.q1);
  const int G = a.group;

  // Block-table entries of a tile, read one tile ahead of their use by a
  // vector load: lane l of every wave reads the entry of sub-tile l / 16
  // (keys kb + 16 (l / 16) .. +15; a 16-key sub-tile never straddles a block,
  // bs >= 16).  A scalar load would share its wait counter with the LDS reads
  // of the key loop; this one is covered by the wait for the tile's DMA.
  const int64_t bmask = PAGED ? ((int64_t)1 << a.idx.bs_log2) - 1 : 0;
  const int32_t* bt_row = PAGED ? a.idx.block_tables + (int64_t)seq * a.idx.bt_stride : nullptr;
  const int num_blocks32 = PAGED ? (int)min(a.idx.num_blocks, (int64_t)0x7fffffff) : 0;
  auto entry_load = [&](int kb) -> int32_t {
    if constexpr (PAGED) {
      const int blk = (kb + 16 * kg) >> a.idx.bs_log2;
      return bt_row[blk < a.idx.max_blocks ? blk : 0];
    } else {
      return 0;
    }
  };
  // (the entries of the first two tiles go out first, with q's loads; the
  // block index is clamped to the row, so the loads stay in the table)
  const int32_t e_tile0 = entry_load(0), e_tile1 = entry_load(kBN);

  // Query rows of this wave: row tile rt covers rows (kRowTiles*wave + rt)*16 + 0..15.
  // q's loads go out before the rows' visibility is worked out and the
  // first tile is requested; q is converted after both (one round trip),
  // except where q is split (QSPLIT: fp32 q held raw across the first
  // tile's set-up spilled), which converts it at once.
  Q32Raw qraw[kRowTiles];
  bool q_ok[kRowTiles];
  float qf[kRowTiles][32];
  float qmax = 0.0f;
  auto convert_q = [&]() {
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
      if (q_ok[rt]) {
        q32_convert(a.q_dtype, qraw[rt], qf[rt]);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) qf[rt][i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) qmax = fmaxf(qmax, fabsf(qf[rt][i]));
    }
  };
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    const int row = (kRowTiles * wave + rt) * 16 + c;
    const int64_t tok = q0 + row / G;
    int d0 = 32 * kg;
    q_ok[rt] = row < a.tok_per_wg * G && tok < q1;
    if constexpr (PAIR) q_ok[rt] = q_ok[rt] && q_slice<PAIR>(G, row % G, kg, d0);
    if (q_ok[rt]) {
      const int hq = kvh * G + row % G;
      q32_issue(a.q, a.q_dtype, (tok * a.num_heads + hq) * kQDim<PAIR> + d0, qraw[rt]);
    }
  }
  // head pairing: this lane's row belongs to the pair's second KV head
  const bool row_hi = PAIR && (kRowTiles * wave * 16 + c) % G >= (G >> 1);
  if constexpr (QSPLIT) convert_q();
  wg_rows<PAGED>(a, vis_lds, red_lds, wk);
  const int min_vis = wk.min_vis, max_vis = wk.max_vis;
  int vis_c[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    const int row = (kRowTiles * wave + rt) * 16 + c;
    vis_c[rt] = PAGED ? vis_lds[row] : row_vis_contiguous(a, wk, row);
  }
  f32x4 acc[kRowTiles][8];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) acc[rt][mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[kRowTiles], l_run[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    m_run[rt] = kNegBig;
    l_run[rt] = 0.0f;
  }
  // The softmax denominators: where P is one fp16 term (FP8 per-tensor and
  // fp16 caches), a ninth output tile O += P . 1 accumulates each row's sum of
  // P on the MFMA units (the same P as the output, rescaled with it): 2 MFMAs
  // per tile in place of 16 VALU adds (FP8 chunks -2.3%).  The bf16 split P
  // would take 4 (+2.7%), and per-token-head caches fold V scales into P, so
  // those sums stay on the VALU (l_run) over the unscaled P.
  constexpr bool kSumMfma = !kTokScale && CT == MKV_DTYPE_F16;
  f32x4 acc_sum[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) acc_sum[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  Op16<CT> ones_op;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (CT == MKV_DTYPE_BF16)
      ones_op[j] = (__bf16)1.0f;
    else
      ones_op[j] = (_Float16)1.0f;
  }

  // K/V staging.  A 16-key sub-tile never straddles a cache block (block
  // size >= 16), so every 16-byte load instruction reads one sub-tile through
  // a wave-uniform buffer descriptor (one scalar block-table lookup); the
  // per-lane offsets are loop-invariant, and keys at or past max_vis, or in
  // an absent block, read zeros (P is 0 there and V must stay finite).
  // The 8 sub-tiles of a tile (K 0-3, V 4-7) are dealt to the workgroup's
  // lanes in slots of 16 keys x kChunks chunks: slot = u * kSlotsPerLoad +
  // tid / kLanesPerSlot for load u; lane: key tid%kLanesPerSlot/kChunks,
  // chunk tid%kChunks.
  constexpr int kLanesPerSlot = 16 * kChunksG;               // 256 (16-bit) / 128 (FP8)
  constexpr int kSlotsPerLoad = kPfThreads / kLanesPerSlot;
  constexpr int kLoads = 8 / kSlotsPerLoad;
  const int64_t row_stride = (int64_t)a.num_kv_heads * kHeadDim * kEbG;
  const int64_t head_bytes = (int64_t)kvh * kHeadDim * kEbG;
  const int ld_key = (tid % kLanesPerSlot) / kChunksG;
  const int ld_ch = tid % kChunksG;
  const uint32_t ld_off = (uint32_t)(ld_key * row_stride + 16 * ld_ch);
  int ld_slot[kLoads];  // wave-uniform
#pragma unroll
  for (int u = 0; u < kLoads; ++u)
    ld_slot[u] = __builtin_amdgcn_readfirstlane(u * kSlotsPerLoad + tid / kLanesPerSlot);
  // LDS offsets of the loads: one per-lane base plus a wave-uniform row
  // shift of 16 (ld_slot[u] & 3) - (ld_slot[0] & 3) keys (the swizzle has
  // period 16), so only the base lives through the loop.  An FP8 chunk
  // (16 elements) becomes two fp16 chunks, written as 2ch + b, then
  // 2ch + 1 - b, with b = ((ch >> 2) ^ key) & 1: LDS writes go 8 lanes (one
  // key) at a time over 32 banks, and b gives those lanes 8 distinct chunk
  // positions mod 8 (and a 16-lane pair of keys all 16).
  const int lds_key0 = 16 * (ld_slot[0] & 3) + ld_key;
  const int ld_b = ((ld_ch >> 2) ^ ld_key) & 1;
  const int lds_base = kEbG == 2 ? LT::offset(lds_key0, ld_ch) : LT::offset(lds_key0, 2 * ld_ch + ld_b);
  const int lds_base2 = kEbG == 2 ? 0 : LT::offset(lds_key0, 2 * ld_ch + 1 - ld_b);
  const uint64_t ld_b_mask = __builtin_amdgcn_ballot_w64(ld_b != 0);  // lanes whose first write is half 1
  auto lds_shift = [&](int u) { return ((ld_slot[u] & 3) - (ld_slot[0] & 3)) * 16 * LT::kRowBytes; };

  // The entries of the tile at kb, validated: per lane (sub-tile l / 16) the
  // physical block (-1 if absent), the byte offset of the sub-tile's first
  // token slot of the sub-tile's first key (paged) and the per-token-head
  // scale index of key kb + l % 64; per wave the tile's first key and its
  // present sub-tiles as bits.
  struct SubTiles {
    int32_t phys;
    uint32_t row;
    int64_t sidx;
    int kb;
    uint32_t present;
  };
  auto entry_use = [&](int kb, int32_t e) -> SubTiles {
    const int t0 = kb + 16 * kg;
    SubTiles st;
    st.kb = kb;
    if constexpr (PAGED) {
      const bool ok = (t0 >> a.idx.bs_log2) < a.idx.max_blocks && e >= 0 && e < num_blocks32;
      st.phys = ok ? e : -1;
      // (the pool holds at most 2^32 token slots)
      st.row = ((uint32_t)e << a.idx.bs_log2) + (uint32_t)(t0 & (int)bmask);
      // (head pairing: threads 128-255 load the scales of the pair's second KV head)
      st.sidx = (int64_t)((uint64_t)(st.row + (uint32_t)(lane & 15)) * (uint64_t)a.scale_heads) +
                (PAIR ? 2 * kvh + ((tid >> 7) & 1) : kvh);
      const uint64_t b = __builtin_amdgcn_ballot_w64(ok);  // bits 16j: sub-tile j
      st.present = (uint32_t)((b & 1u) | ((b >> 15) & 2u) | ((b >> 30) & 4u) | ((b >> 45) & 8u));
    } else {
      st.phys = 0;
      st.row = 0;
      st.sidx = 0;
      st.present = 0xfu;
    }
    return st;
  };
  // Descriptor of rows 16j .. 16j+15 of one tensor's tile (no records when
  // the sub-tile's block is absent: its loads read zeros).  The byte offset
  // is formed in scalar registers from the sub-tile's first row (lane 16j's
  // slot, or the sequence's row for contiguous K/V), only in the waves that
  // issue loads.
  auto sub_rsrc = [&](const char* base, const SubTiles& st, int j) -> __amdgpu_buffer_rsrc_t {
    int64_t r64;
    if constexpr (PAGED)
      r64 = (uint32_t)__builtin_amdgcn_readlane((int)st.row, 16 * j);
    else
      r64 = q_seq0 + st.kb + 16 * j;
    const int64_t off = r64 * row_stride + head_bytes;
    const int num = (st.present >> j) & 1u ? (int)(15 * row_stride + kHeadDim * kEbG) : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, num, 0x00020000);
  };
  // 16-bit caches: tiles go straight from HBM into LDS (buffer_load ... lds,
  // 16 bytes per lane, no registers, no LDS write instructions).  One wave's
  // load fills 1 KB = 4 key rows contiguously, lane l at byte 16l (key row
  // l / 16, stored chunk l % 16), so lane l reads logical chunk
  // (l % 16) ^ s(key) of its key; s has period 16 and each load's 4 rows
  // start at a multiple of 4, so the offset is the same for every load.
  // Waves 0-3 stage the whole tile (wave w: rows 4w .. 4w+3 of each of the
  // 8 sub-tiles, K 0-3 then V 0-3); waves 4-7 skip the descriptors and the
  // issue (2-3% faster than 4 loads in every wave: the loop is VALU-bound and
  // waves w and w + 4 share a SIMD).
  static_assert(!kDma || (kSlotsPerLoad == 2 && kLoads == 4), "DMA slot layout");
  const uint32_t ld_off_dma = (uint32_t)(ld_key * row_stride + 16 * (ld_ch ^ LT::swz(ld_key)));
  const int dma_row = __builtin_amdgcn_readfirstlane(4 * (wave & 3) * LT::kRowBytes);
  auto dma_tile = [&](int kb, const SubTiles& st, int buf) {
    if (wave >= 4) return;  // waves 0-3 stage the whole tile
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = u & 3;  // K sub-tiles 0-3, then V sub-tiles 0-3
      const int t0 = kb + 16 * j;
      const __amdgpu_buffer_rsrc_t r = sub_rsrc(u >= 4 ? a.v : a.k, st, j);
      const uint32_t off = ld_key < max_vis - t0 ? ld_off_dma : 0x80000000u;
      char* dst = (u >= 4 ? VBUF(buf) : KBUF(buf)) + 16 * j * LT::kRowBytes + dma_row;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, 0);
    }
  };
  u32x4 stg[kLoads];
  // Per-token-head scales of a tile: lane tid < 128 loads the K (tid % 128 <
  // 64) or V scale of key tid % 64, and with head pairing lanes 128-255 the
  // same for the pair's second KV head (0 for keys past max_vis or in absent
  // blocks; every lane loads, the others from index 0, so the load is
  // unconditional).
  constexpr int kScLoads = PAIR ? 256 : 128;
  float stg_sc = 0.0f;
  auto load_scales = [&](int kb, const SubTiles& st) {
    if constexpr (kTokScale && PAGED) {
      // lane tid % 64 holds key kb + tid % 64 (sub-tile (tid % 64) / 16)
      const bool valid = tid < kScLoads && st.phys >= 0 && kb + (tid & 63) < max_vis;
      const float* base = (PAIR ? (tid & 64) != 0 : tid >= 64) ? a.v_scale : a.k_scale;
      const float x = base[valid ? st.sidx : 0];
      stg_sc = valid ? x : 0.0f;
    }
  };
  auto load_tile = [&](int kb, const SubTiles& st) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int j = ld_slot[u] & 3;
      const bool is_v = ld_slot[u] >= 4;
      const int64_t t0 = kb + 16 * j;
      const __amdgpu_buffer_rsrc_t r = sub_rsrc(is_v ? a.v : a.k, st, j);
      const uint32_t off = (t0 + ld_key < max_vis) ? ld_off : 0x80000000u;
      stg[u] = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    }
    load_scales(kb, st);
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const bool is_v = ld_slot[u] >= 4;
      char* dst = (is_v ? VBUF(buf) : KBUF(buf)) + lds_shift(u);
      if constexpr (kEbG == 2) {
        *reinterpret_cast<u32x4*>(dst + lds_base) = stg[u];
      } else {
        // e4m3 / int8 -> fp16 is exact; elements 8h .. 8h+7 of the chunk
        // from dwords 2h, 2h+1
        auto pair = [&](uint32_t d, auto hi_tag) -> uint32_t {
          constexpr bool kHi = decltype(hi_tag)::value;
          if constexpr (KV_DT == kKvI8PerToken)
            return __builtin_bit_cast(uint32_t, i8x2_to_f16x2<kHi>(d));
          else
            return __builtin_bit_cast(uint32_t, fp8x2_to_f16x2<kHi>(d));
        };
        // (the lane's first write takes half ld_b: one v_cndmask per dword
        // on the lanes' ld_b mask; written as selects in C++, LLVM turns them
        // into an index 2 * ld_b, a 4-way select per dword)
        auto half = [&](uint32_t d0, uint32_t d1) {
          return u32x4{pair(d0, std::false_type{}), pair(d0, std::true_type{}),
                       pair(d1, std::false_type{}), pair(d1, std::true_type{})};
        };
        *reinterpret_cast<u32x4*>(dst + lds_base) =
            half(lane_select(stg[u][0], stg[u][2], ld_b_mask), lane_select(stg[u][1], stg[u][3], ld_b_mask));
        *reinterpret_cast<u32x4*>(dst + lds_base2) =
            half(lane_select(stg[u][2], stg[u][0], ld_b_mask), lane_select(stg[u][3], stg[u][1], ld_b_mask));
      }
    }
    if constexpr (kTokScale) {
      if (tid < kScLoads) sc_lds[buf * kScPerBuf + tid] = stg_sc;
      // the waves holding V scales (tid & 64; with head pairing one per KV
      // head) also store the tile's largest one
      if (tid < kScLoads && (tid & 64)) {
        const float vm = wave_max_dpp(stg_sc);
        if (lane == 0) vmax_lds[2 * buf + (tid >> 7)] = vm;
      }
    }
  };

  // Transposed V reads.  ds_read_b64_tr_b16: within each 16-lane group, lane
  // d receives element d%4 of the 8-byte reads of lanes 4i + d/4 (i = 0..3).
  // So if lane 4i + q of lane group kg reads key 4kg + i at dims 16mm + 4q,
  // lane c receives V[4kg + i][16mm + c] for the lane group's MFMA k-slice,
  // where the P operand holds keys 32ks + 16*(j/4) + 4kg + j%4 (the second
  // half j >= 4 reads 16 rows further).  The offsets follow from two
  // per-lane values (computed where they are used, so they do not hold eight
  // registers through the key loop): chunk (2mm + x) ^ s =
  // ((mm ^ (s >> 1)) << 1) | (x ^ (s & 1)), hence offset(mm) = vt_base +
  // ((mm << 5) ^ vt_swh).
  int vt_base, vt_swh;
  {
    const int s16 = lane & 15;
    const int i = s16 >> 2, q = s16 & 3;
    const int key = 4 * kg + i;
    const int sw = LT::swz(key);
    vt_base = key * LT::kRowBytes + ((((q >> 1) ^ sw) & 1) << 4) + 8 * (q & 1);
    vt_swh = (sw >> 1) << 5;
    // one opaque value: split into its terms, the address of a V read became
    // a chain of GEPs too deep for the LDS alias-scope annotation, and a read
    // without it waits for every pending LDS DMA
    if constexpr (kDma) asm volatile("" : "+v"(vt_base));
  }

  const int n_tiles = (max_vis + kBN - 1) / kBN;
  // A wave whose rows see no key (padding rows: the workgroup of a short
  // chunk, e.g. a decode row of a mixed batch, whose G rows sit in wave 0)
  // still loads its share of every tile and meets every barrier, but skips
  // the math.
  bool wave_rows = false;
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) wave_rows |= vis_c[rt] > 0;
  const bool wave_active = __builtin_amdgcn_ballot_w64(wave_rows) != 0;
  // present sub-tiles of the current and the next tile; raw entries of the
  // tile after the next (in flight)
  uint32_t present_cur = 0xfu, present_nxt = 0xfu;
  int32_t e_ahead = 0;
  // The first tile's loads go out before q is waited for and converted
  // below, so that the two round trips overlap (q waited for first, then the
  // tile, took ~0.6 us more per workgroup).
  if (n_tiles > 0) {
    const SubTiles st0 = entry_use(0, e_tile0);
    present_cur = st0.present;
    e_ahead = e_tile1;
    if constexpr (kDma)
      dma_tile(0, st0, 0);
    else
      load_tile(0, st0);
  }
  if constexpr (!QSPLIT) convert_q();
  float score_mul = a.sm_scale * kLog2e;
  if constexpr (KV_DT == MKV_DTYPE_FP8E4M3) score_mul *= load_uniform_f32(a.k_scale);
  if constexpr (CT != MKV_DTYPE_BF16) {
    // power-of-two normalisation so that q is exact and in range in fp16
    qmax = wave_max_dpp(qmax);
    if (qmax > 0.0f && qmax < __builtin_huge_valf()) {
      const int e = ilogbf(qmax);
      const float f = ldexpf(1.0f, 8 - e);
#pragma unroll
      for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
        for (int i = 0; i < 32; ++i) qf[rt][i] *= f;
      score_mul *= ldexpf(1.0f, e - 8);
    }
  }
  // The loop keeps raw scores and needs score_mul > 0: a negative scale
  // moves its sign into q (exact), a zero scale is q = 0 with scale 1 (every
  // visible key weighs the same, as with 0 * score); NaN propagates.
  if (!(score_mul > 0.0f) && score_mul == score_mul) {
    const float f = score_mul < 0.0f ? -1.0f : 0.0f;
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
      for (int i = 0; i < 32; ++i) qf[rt][i] *= f;
    score_mul = score_mul < 0.0f ? -score_mul : 1.0f;
  }
  Op16<CT> qop[kRowTiles][4];
  Op16<CT> qlo[QSPLIT ? kRowTiles : 1][4];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      qop[rt][st] = to_op16<CT>(qf[rt] + 8 * st);
      if constexpr (QSPLIT) {
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = qf[rt][8 * st + j] - (float)qop[rt][st][j];
        qlo[rt][st] = to_op16<CT>(r);
      }
    }

  if (n_tiles > 0) {
    if constexpr (kDma)
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    else
      store_tile(0);
  }
  __syncthreads();
  __builtin_amdgcn_s_setprio(0);
  // Two tiles per trip (the inner loop unrolls fully), so that each buffer
  // index is a compile-time constant (LDS addresses fold into the read and
  // write offsets).
  constexpr int kPerTrip = 2;
  for (int it0 = 0; it0 < n_tiles; it0 += kPerTrip) {
#pragma unroll
  for (int h = 0; h < kPerTrip; ++h) {
    const int it = it0 + h;
    if (it >= n_tiles) break;
    const int buf = h;
    const int kb = it * kBN;
    if (it + 1 < n_tiles) {
      const SubTiles st1 = entry_use(kb + kBN, e_ahead);
      present_nxt = st1.present;
      if constexpr (kDma)
        dma_tile(kb + kBN, st1, buf ^ 1);
      else
        load_tile(kb + kBN, st1);
      e_ahead = entry_load(kb + 2 * kBN);
    }
    if (wave_active) {

    // Key sub-tile validity (16 keys never straddle a block: bs >= 16).
    bool kvalid[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) kvalid[kt] = (present_cur >> kt) & 1u;
    const bool full = kb + kBN <= min_vis && kvalid[0] && kvalid[1] && kvalid[2] && kvalid[3];

    // ---- S^T = K Q^T ----
    // The MFMA blocks run at raised wave priority: a SIMD's waves reach the
    // same phase together (one barrier per tile), and issuing the MFMAs of
    // whichever waves have them first keeps the matrix pipe fed while the
    // other waves' softmax fills the gaps.
    __builtin_amdgcn_s_setprio(1);
    // 16-bit: the lane's key row, recomputed here: held across the loop it
    // is the register the allocator spills first, and its reload would wait
    // for the tile prefetch issued just above.
    const int c_k = lane_id_volatile() & 15;
    f32x4 s[4][kRowTiles];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int rt = 0; rt < kRowTiles; ++rt) s[kt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int key = 16 * kt + c_k;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(KBUF(buf) + LT::offset(key, 4 * kg + st));
        const Op16<CT> kop = __builtin_bit_cast(Op16<CT>, w);
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          s[kt][rt] = mfma16<CT>(kop, qop[rt][st], s[kt][rt]);
          if constexpr (QSPLIT) s[kt][rt] = mfma16<CT>(kop, qlo[rt][st], s[kt][rt]);
        }
      }
    }

    __builtin_amdgcn_s_setprio(0);
    // ---- online softmax (log2 domain), per row = lane column c ----
    // The scores stay unscaled (score_mul > 0): the max of the scaled scores
    // is the scaled max of the raw ones (rounding a product by a positive
    // constant is monotonic), and each P takes one FMA.
    float l_scaled[kRowTiles];
    // Per-token-head V scales fold into P, which must stay below the fp16
    // maximum: P <= 2^8 (the lazy rescale), so a tile whose largest V scale
    // is 2^e times a fraction in [1/2, 1) with e > 7 lifts the max it offers
    // the running max by e - 7 (log2 units), which keeps P * v_scale <= 2^15.
    // Any offset of the running max cancels in the normalisation; with every
    // V scale below 128 (FP8 amax < 57344, INT8 amax < 16256) it is 0.
    // (The scale is the same in every lane: its exponent is taken from the
    // bits in scalar registers, e = biased exponent - 126, so the lift holds
    // no vector register through the softmax.)
    float v_lift = 0.0f;
    if constexpr (kTokScale) {
      float vm = vmax_lds[2 * buf];
      if constexpr (PAIR) vm = fmaxf(vm, vmax_lds[2 * buf + 1]);
      const int e = ((__builtin_amdgcn_readfirstlane(__float_as_int(vm)) >> 23) & 0xff) - 126;
      v_lift = e > 7 ? (float)(e - 7) : 0.0f;
    }
    // per-token-head K scales of this lane's keys 16kt + 4kg + r
    if constexpr (kTokScale) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const f32x4 ksc =
            *reinterpret_cast<const f32x4*>(sc_lds + buf * kScPerBuf + (row_hi ? 128 : 0) + 16 * kt + 4 * kg);
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[kt][rt][r] *= ksc[r];
      }
    }
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
      if (!full) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = kb + 16 * kt + 4 * kg + r;
            if (!(t < vis_c[rt] && kvalid[kt])) s[kt][rt][r] = -__builtin_huge_valf();
          }
      }
      float mx = -__builtin_huge_valf();
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][rt][r]);
      mx = max_xor32(max_xor16(mx));
      mx = fmaxf(mx * score_mul, kNegBig) + v_lift;
      // Lazy rescale: the running max only moves when the tile's max exceeds
      // it by more than kRescaleSlack (log2 units), so P <= 2^kRescaleSlack,
      // exact and in range in bf16/fp16; the output rescale below then runs
      // only in a row's first tiles.  The result is the same softmax.
      const float m_new = mx > m_run[rt] + kRescaleSlack ? mx : m_run[rt];
      const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_new);
      m_run[rt] = m_new;
      l_scaled[rt] = l_run[rt] * alpha;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * kg + r);
#pragma unroll
          for (int mm = 0; mm < 8; ++mm) acc[rt][mm][r] *= ar;
          if constexpr (kSumMfma) acc_sum[rt][r] *= ar;
        }
      }
    }

    // ---- P = exp2(score - m) and O += P V, 32 keys per MFMA k-step ----
    // B operand of output-dim tile mm (dims 16mm .. 16mm+15, lane c -> dim
    // 16mm + c): the lane group's 8 keys of its k-slice, read transposed
    // straight from LDS (ds_read_b64_tr_b16, see vt_base above).
    char* vbuf = VBUF(buf);
    // (a lambda: written inline, the same step leaves the compiler's register
    // allocation spilling in the per-token-head variants)
    auto pv_step = [&](auto split_tag) {
    constexpr bool kSplitP = decltype(split_tag)::value;
    float p[4][kRowTiles][4];
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
      const float m_new = m_run[rt];
      float psum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kt][rt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][rt][r], score_mul, -m_new));
          if constexpr (!kSumMfma) psum = (kt | r) ? psum + p[kt][rt][r] : p[kt][rt][r];
        }
      if constexpr (!kSumMfma) l_run[rt] = l_scaled[rt] + psum;
      if constexpr (kTokScale) {
        // per-token-head V scales of keys 16kt + 4kg + r, folded into P
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const f32x4 vs = *reinterpret_cast<const f32x4*>(sc_lds + buf * kScPerBuf + (row_hi ? 128 : 0) + 64 +
                                                           16 * kt + 4 * kg);
#pragma unroll
          for (int r = 0; r < 4; ++r) p[kt][rt][r] *= vs[r];
        }
      }
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Op16<CT> pop[kRowTiles], plop[kRowTiles];
#pragma unroll
      for (int rt = 0; rt < kRowTiles; ++rt) {
        float pv[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = p[2 * ks][rt][r];
          pv[4 + r] = p[2 * ks + 1][rt][r];
        }
        pop[rt] = to_op16<CT>(pv);
        if constexpr (CT == MKV_DTYPE_BF16) {
        if constexpr (kSplitP) {
          // second bf16 term carrying P's rounding residual (~16-bit P);
          // p - hi is exact in fp32 and one dot2 forms it: hi_pair . (-1, 0)
          // + p for the even element, . (0, -1) + p for the odd one.  The
          // two constants are bit patterns held in scalar registers (an
          // inline float constant is not a bf16 pair).
          typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
          uint32_t nl_bits = 0x0000bf80u, nh_bits = 0xbf800000u;
          asm volatile("" : "+s"(nl_bits), "+s"(nh_bits));
          const bf16x2 neg_lo = __builtin_bit_cast(bf16x2, nl_bits), neg_hi = __builtin_bit_cast(bf16x2, nh_bits);
          float plo[8];
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const bf16x2 h = {pop[rt][j], pop[rt][j + 1]};
            plo[j] = __builtin_amdgcn_fdot2_f32_bf16(h, neg_lo, pv[j], false);
            plo[j + 1] = __builtin_amdgcn_fdot2_f32_bf16(h, neg_hi, pv[j + 1], false);
          }
          plop[rt] = to_op16<CT>(plo);
        }
        }
      }
      // all 8 B operands read ahead of their MFMAs so that the LDS reads overlap
      Op16<CT> Bv[8];
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
        typedef short v4i16 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
        const int vo = vt_base + ((mm << 5) ^ vt_swh);
        lds_v4i16* p0 = (lds_v4i16*)(vbuf + vo + 32 * ks * LT::kRowBytes);
        lds_v4i16* p1 = (lds_v4i16*)(vbuf + vo + (32 * ks + 16) * LT::kRowBytes);
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0);
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1);
        const u32x4 w = {(uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16),
                         (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16),
                         (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16),
                         (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16)};
        Bv[mm] = __builtin_bit_cast(Op16<CT>, w);
      }
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          acc[rt][mm] = mfma16<CT>(pop[rt], Bv[mm], acc[rt][mm]);
          if constexpr (CT == MKV_DTYPE_BF16) {
            if constexpr (kSplitP) acc[rt][mm] = mfma16<CT>(plop[rt], Bv[mm], acc[rt][mm]);
          }
        }
      }
      if constexpr (kSumMfma) {
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          acc_sum[rt] = mfma16<CT>(pop[rt], ones_op, acc_sum[rt]);
          if constexpr (CT == MKV_DTYPE_BF16) {
            if constexpr (kSplitP) acc_sum[rt] = mfma16<CT>(plop[rt], ones_op, acc_sum[rt]);
          }
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    };
    pv_step(std::bool_constant<CT == MKV_DTYPE_BF16>{});
    }  // wave_active

    if constexpr (kDma)
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's DMA has landed
    else if (it + 1 < n_tiles)
      store_tile(buf ^ 1);
    present_cur = present_nxt;
    __syncthreads();
  }
  }

#undef KBUF
#undef VBUF
  __builtin_amdgcn_s_setprio(3);
  {
  // the lane's indices again, recomputed here rather than held in registers
  // across the key loop (held, they were spilled to scratch)
  const int lane = lane_id_volatile();
  const int c = lane & 15, kg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // ---- normalise and write rows 4kg + r of each row tile ----
  const float v_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.v_scale) : 1.0f;
  static_assert(kRowTiles == 1, "the staged epilogue holds one 16-row tile per wave");
  if (a.q_dtype != MKV_DTYPE_F32) {
    // 16-bit outputs: the wave's 16 x 128 tile is staged in LDS (free after
    // the last tile's barrier; 16 rows of 272 bytes per wave, two waves per
    // 16 KB tile buffer: the 16-byte row padding puts the four rows of a
    // write on distinct banks and makes each element's address the row's
    // base plus an immediate) and written as whole 16-byte chunks, 4 stores
    // per lane instead of 32 two-byte ones.
    constexpr int kStageRow = 272;
    static_assert(!kDma || 2 * 16 * kStageRow <= kSplitBytes, "two waves' staging per tile buffer");
    static_assert(kDma || kPfWaves * 16 * kStageRow <= kOneBytes, "every wave's staging in the tile array");
    static_assert(kRowsPerWg <= 128, "row / G by multiply-shift holds for rows below 128");
    char* stage;
    if constexpr (kDma) {
      char* const half = wave < 4 ? (wave < 2 ? lds_k0 : lds_v0) : (wave < 6 ? lds_k1 : lds_v1);
      stage = half + (wave & 1) * 16 * kStageRow;
    } else {
      stage = lds_kv + wave * 16 * kStageRow;
    }
    // 1 / l of rows 4kg + r: one division per lane (its own row c, then
    // moved) where the sums are on the VALU; the MFMA row sums hold row
    // 4kg + r in every lane of the group.
    float inv_r[4];
    if constexpr (kSumMfma) {
#pragma unroll
      for (int r = 0; r < 4; ++r) inv_r[r] = acc_sum[0][r] > 0.0f ? v_mul / acc_sum[0][r] : 0.0f;
    } else {
      float l_col = l_run[0] + __shfl_xor(l_run[0], 16);
      l_col += __shfl_xor(l_col, 32);
      const float inv_c = l_col > 0.0f ? v_mul / l_col : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) inv_r[r] = __shfl(inv_c, 4 * kg + r);
    }
    char* const wbase = stage + 4 * kg * kStageRow + 2 * c;  // + r rows + 32 bytes per output tile
    if (a.q_dtype == MKV_DTYPE_BF16) {
      typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int mm = 0; mm < 8; mm += 2) {
          // round to nearest even, two elements per conversion
          const bf16x2_t h = {(__bf16)(acc[0][mm][r] * inv_r[r]), (__bf16)(acc[0][mm + 1][r] * inv_r[r])};
          const uint32_t pk = __builtin_bit_cast(uint32_t, h);
          *reinterpret_cast<uint16_t*>(wbase + r * kStageRow + 32 * mm) = (uint16_t)pk;
          *reinterpret_cast<uint16_t*>(wbase + r * kStageRow + 32 * (mm + 1)) = (uint16_t)(pk >> 16);
        }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int mm = 0; mm < 8; ++mm)
          *reinterpret_cast<uint16_t*>(wbase + r * kStageRow + 32 * mm) =
              (uint16_t)f32_to_f16_bits(acc[0][mm][r] * inv_r[r]);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's staging writes are done
    __builtin_amdgcn_wave_barrier();
    // row / G for row < 128 and G <= 128: (row * gm) >> 16 with
    // gm = 65536 / G + 1 (the excess, below 128 / 65536, stays under 1 / G)
    const uint32_t gm = 65536u / (uint32_t)G + 1u;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rr = 4 * u + kg, ch = c;  // chunk 64u + lane: row rr, 16-byte chunk ch
      const int row = 16 * wave + rr;
      const int rq = (int)(((uint32_t)row * gm) >> 16);
      const int64_t tok = q0 + rq;
      const u32x4 d = *reinterpret_cast<const u32x4*>(stage + rr * kStageRow + 16 * ch);
      int col0;
      if (row < a.tok_per_wg * G && tok < q1 && out_cols<PAIR>(G, row - rq * G, ch, col0)) {
        const int hq = kvh * G + (row - rq * G);
        st16(reinterpret_cast<uint16_t*>(a.out) + (tok * a.num_heads + hq) * kQDim<PAIR> + col0, d);
      }
    }
    return;
  }
  // fp32 outputs: 1 / l as above; row / G by the multiply-shift below (a
  // division by G here would keep the divider's reciprocal in a register
  // across the key loop)
  const uint32_t gm32 = 65536u / (uint32_t)G + 1u;
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    float inv_r[4];
    if constexpr (kSumMfma) {
#pragma unroll
      for (int r = 0; r < 4; ++r) inv_r[r] = acc_sum[rt][r] > 0.0f ? v_mul / acc_sum[rt][r] : 0.0f;
    } else {
      float l_col = l_run[rt] + __shfl_xor(l_run[rt], 16);
      l_col += __shfl_xor(l_col, 32);
      const float inv_c = l_col > 0.0f ? v_mul / l_col : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) inv_r[r] = __shfl(inv_c, 4 * kg + r);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = (kRowTiles * wave + rt) * 16 + 4 * kg + r;
      const int rq = (int)(((uint32_t)row * gm32) >> 16), rm = row - rq * G;
      const int64_t tok = q0 + rq;
      if (row >= a.tok_per_wg * G || tok >= q1) continue;
      const int hq = kvh * G + rm;
      // lane c holds dims 16mm + c (head pairing: a row keeps dims 64 hi ..
      // 64 hi + 63, i.e. mm = 4 hi .. 4 hi + 3)
      const bool hi = PAIR && rm >= (G >> 1);
      const int64_t o = (tok * a.num_heads + hq) * kQDim<PAIR> + c - (hi ? 64 : 0);
#pragma unroll
      for (int mm = 0; mm < 8; ++mm)
        if (!PAIR || (mm >= 4) == hi) reinterpret_cast<float*>(a.out)[o + 16 * mm] = acc[rt][mm][r] * inv_r[r];
    }
  }
  }
}

template <int KV_DT, bool PAGED, bool QSPLIT, bool PAIR>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(4))) void prefill_mfma_kernel(PrefillArgs a) {
  prefill_mfma_body<KV_DT, PAGED, QSPLIT, PAIR>(a);
}

// The variants that do not fit four waves per SIMD without spilling (the
// per-token-head formats with a split q, or with head pairing, which holds
// a second scale set per key) run at two waves per SIMD, one workgroup per
// CU, with up to 256 registers.
template <int KV_DT, bool PAGED, bool QSPLIT, bool PAIR>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2))) void prefill_mfma_2w_kernel(PrefillArgs a) {
  prefill_mfma_body<KV_DT, PAGED, QSPLIT, PAIR>(a);
}

template <int KV_DT, bool QSPLIT, bool PAIR>
constexpr bool kPrefill2w = kPerTokenScale<KV_DT> && (QSPLIT || PAIR);

// ---------------------------------------------------------------------------
// fp32 caches (the reference engine's default precision, model_runner.py:87,
// :249; flash_attention_prefill / paged_attention_prefill_triton take fp32,
// attention.py:446-514, :852-891).  The same work decomposition as
// prefill_mfma_kernel (128 rows of one sequence and KV head per workgroup,
// the same tile list), on the fp32 MFMA (v_mfma_f32_16x16x4_f32: products
// and sums in fp32, no rounding of K, V, q or P below fp32).
//
// Tiles of kBN32 = 32 keys x 512 bytes go from HBM straight into LDS by DMA
// (buffer_load ... lds), double-buffered.  Wave w loads 8 consecutive keys
// of one 16-key sub-tile: K (w < 4) or V, sub-tile (w % 4) / 2, keys
// 8 (w % 2) .. +7, two key rows per instruction.  K rows are stored with
// 16-byte chunk p holding logical chunk p ^ (key & 15) (the swizzle moves to
// the global side of the DMA), so that the 16 lanes of a QK operand read
// (16 keys, one logical chunk) hit 16 distinct chunk positions mod 16; V rows
// are stored as they are (the 16 lanes of a PV operand read take one key's
// chunks c and 16 + c).
//
// Per wave (16 rows), per 16-key sub-tile kt:
//   S^T = K Q^T: 32 MFMAs; lane (c, kg) supplies K[key c][32 kg + st] and
//     q[row c][32 kg + st] at step st (the contraction order over head_dim
//     is free), and receives S^T[key 4 kg + r][row c].
//   O += P V: 4 x 8 MFMAs; step r takes P[row c][key 4 kg + r] (from the
//     lane's own scores) and V[key 4 kg + r][dim], where output tile mm and
//     lane column c hold dim 4c + mm (mm < 4) or 64 + 4c + mm - 4.
// ---------------------------------------------------------------------------
constexpr int kBN32 = 32;
constexpr int kRowBytes32 = kHeadDim * 4;          // 512
constexpr int kTileBytes32 = kBN32 * kRowBytes32;  // 16 KB per K or V tile

template <bool PAGED, bool PAIR>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(4))) void prefill_f32_kernel(PrefillArgs a) {
  extern __shared__ __align__(16) char smem[];
  __shared__ __align__(16) char lds_k0[kTileBytes32], lds_v0[kTileBytes32], lds_k1[kTileBytes32],
      lds_v1[kTileBytes32];
  int* vis_lds = reinterpret_cast<int*>(smem);
  int* red_lds = vis_lds + kRowsPerWg;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, kg = lane >> 4;

  WgWork wk;
  if (!wg_tile<PAGED>(a, smem, wk)) return;
  const int kvh = wk.kvh, seq = wk.seq;
  const int64_t q0 = wk.q0, q1 = wk.q1;
  const int G = a.group;

  // q of row c (dims 32 kg .. 32 kg + 31), fp32, loaded before the rows'
  // visibility is worked out
  const int my_row = 16 * wave + c;
  float qf[32];
  {
    const int64_t tok = q0 + my_row / G;
    int d0 = 32 * kg;
    bool ok = my_row < a.tok_per_wg * G && tok < q1;
    if constexpr (PAIR) ok = ok && q_slice<PAIR>(G, my_row % G, kg, d0);
    if (ok) {
      const int hq = kvh * G + my_row % G;
      const int64_t off = (tok * a.num_heads + hq) * kQDim<PAIR> + d0;
      load_q32(a.q, a.q_dtype, off, qf);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) qf[i] = 0.0f;
    }
  }
  wg_rows<PAGED>(a, vis_lds, red_lds, wk);
  const int min_vis = wk.min_vis, max_vis = wk.max_vis;
  const int vis_row = PAGED ? vis_lds[my_row] : row_vis_contiguous(a, wk, my_row);
  // The loop keeps raw scores and needs score_mul > 0 (as prefill_mfma_kernel).
  float score_mul = a.sm_scale * kLog2e;
  if (!(score_mul > 0.0f) && score_mul == score_mul) {
    const float f = score_mul < 0.0f ? -1.0f : 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) qf[i] *= f;
    score_mul = score_mul < 0.0f ? -score_mul : 1.0f;
  }

  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;

  // DMA geometry of this wave: tensor (K for waves 0-3), sub-tile j, first
  // key kw of its 8; lane l fills key kw + 2u + l / 32 at chunk position
  // l % 32 in instruction u.
  const int64_t row_stride = (int64_t)a.num_kv_heads * kRowBytes32;
  const int64_t head_bytes = (int64_t)kvh * kRowBytes32;
  const bool w_is_v = wave >= 4;
  const int w_sub = (wave & 3) >> 1;
  const int w_key = 8 * (wave & 1);
  uint32_t dma_off[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int key = w_key + 2 * u + (lane >> 5);  // within the sub-tile (== key & 15)
    const int p = lane & 31;
    const int gch = w_is_v ? p : (p ^ key);
    dma_off[u] = (uint32_t)(key * row_stride + 16 * gch);
  }
  auto dma_tile = [&](int kb, char* kbuf, char* vbuf) {
    const int64_t t0 = kb + 16 * w_sub;
    const char* base = w_is_v ? a.v : a.k;
    const char* ptr = base;
    int num = 0;
    if constexpr (PAGED) {
      const int64_t phys = a.idx.physical_block(seq, t0 >> a.idx.bs_log2);
      if (phys >= 0) {
        const int64_t bmask = ((int64_t)1 << a.idx.bs_log2) - 1;
        ptr = base + ((phys << a.idx.bs_log2) + (t0 & bmask)) * row_stride + head_bytes;
        num = (int)(15 * row_stride + kRowBytes32);
      }
    } else {
      ptr = base + (wk.q_seq0 + t0) * row_stride + head_bytes;
      num = (int)(15 * row_stride + kRowBytes32);
    }
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)ptr, (short)0, num, 0x00020000);
    char* dst0 = (w_is_v ? vbuf : kbuf) + (16 * w_sub + w_key) * kRowBytes32;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t key = t0 + w_key + 2 * u + (lane >> 5);
      const uint32_t off = key < max_vis ? dma_off[u] : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(dst0 + 2 * u * kRowBytes32), 16, off, 0, 0, 0);
    }
  };
  // validity of the two 16-key sub-tiles of the tile at kb (absent blocks)
  auto sub_valid = [&](int kb, int kt) -> bool {
    if constexpr (PAGED) return a.idx.physical_block(seq, (int64_t)(kb + 16 * kt) >> a.idx.bs_log2) >= 0;
    return true;
  };

  const int n_tiles = (max_vis + kBN32 - 1) / kBN32;
  const bool wave_active = __builtin_amdgcn_ballot_w64(vis_row > 0) != 0;
  if (n_tiles > 0) {
    dma_tile(0, lds_k0, lds_v0);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  }
  __syncthreads();
  for (int it0 = 0; it0 < n_tiles; it0 += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int it = it0 + h;
      if (it >= n_tiles) break;
      char* kbuf = h ? lds_k1 : lds_k0;
      char* vbuf = h ? lds_v1 : lds_v0;
      const int kb = it * kBN32;
      if (it + 1 < n_tiles) dma_tile(kb + kBN32, h ? lds_k0 : lds_k1, h ? lds_v0 : lds_v1);
      if (wave_active) {
        bool kvalid[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) kvalid[kt] = sub_valid(kb, kt);
        const bool full = kb + kBN32 <= min_vis && kvalid[0] && kvalid[1];
        // ---- S^T = K Q^T ----
        f32x4 s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
          const char* krow = kbuf + (16 * kt + c) * kRowBytes32;
#pragma unroll
          for (int qd = 0; qd < 8; ++qd) {
            const f32x4 kv4 = *reinterpret_cast<const f32x4*>(krow + 16 * ((8 * kg + qd) ^ c));
#pragma unroll
            for (int e = 0; e < 4; ++e)
              s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv4[e], qf[4 * qd + e], s[kt], 0, 0, 0);
          }
        }
        // ---- online softmax (log2 domain) for row c ----
        if (!full) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = kb + 16 * kt + 4 * kg + r;
              if (!(t < vis_row && kvalid[kt])) s[kt][r] = -__builtin_huge_valf();
            }
        }
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][r]);
        mx = max_xor32(max_xor16(mx));
        mx = fmaxf(mx * score_mul, kNegBig);
        const float m_new = mx > m_run + kRescaleSlack ? mx : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            s[kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], score_mul, -m_new));
            psum += s[kt][r];
          }
        l_run = l_run * alpha + psum;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * kg + r);
#pragma unroll
            for (int mm = 0; mm < 8; ++mm) acc[mm][r] *= ar;
          }
        }
        // ---- O += P V ----
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const char* vrow = vbuf + (16 * kt + 4 * kg + r) * kRowBytes32;
            const f32x4 v_lo = *reinterpret_cast<const f32x4*>(vrow + 16 * c);
            const f32x4 v_hi = *reinterpret_cast<const f32x4*>(vrow + 256 + 16 * c);
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
              acc[mm] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[kt][r], v_lo[mm], acc[mm], 0, 0, 0);
              acc[4 + mm] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[kt][r], v_hi[mm], acc[4 + mm], 0, 0, 0);
            }
          }
      }  // wave_active
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's DMA has landed
      __syncthreads();
    }
  }

  // ---- normalise and write rows 4 kg + r ----
  // (the lane's indices recomputed rather than held across the key loop, and
  // row / G by multiply-shift for row < 128: no divider kept across it)
  const int lane_e = lane_id_volatile();
  const int ce = lane_e & 15, kge = lane_e >> 4;
  const uint32_t gm = 65536u / (uint32_t)G + 1u;
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float lh = __shfl(l_col, 4 * kge + r);
    const int row = 16 * wave + 4 * kge + r;
    const int rq = (int)(((uint32_t)row * gm) >> 16), rm = row - rq * G;
    const int64_t tok = q0 + rq;
    if (row >= a.tok_per_wg * G || tok >= q1) continue;
    const int hq = kvh * G + rm;
    const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
    float lo[8], hi[8];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      lo[mm] = acc[mm][r] * inv;
      hi[mm] = acc[4 + mm][r] * inv;
    }
    const int64_t o = (tok * a.num_heads + hq) * kQDim<PAIR>;
    // head pairing: a row of the pair's first KV head keeps dims 0-63 (lo),
    // one of its second dims 64-127 (hi), stored at the row's dims 0-63
    const bool row_hi = PAIR && rm >= (G >> 1);
    const bool keep_lo = !PAIR || !row_hi, keep_hi = !PAIR || row_hi;
    const int hi_off = PAIR ? 0 : 64;
    if (a.q_dtype == MKV_DTYPE_F32) {
      float* po = reinterpret_cast<float*>(a.out) + o;
      if (keep_lo) *reinterpret_cast<f32x4*>(po + 4 * ce) = f32x4{lo[0], lo[1], lo[2], lo[3]};
      if (keep_hi) *reinterpret_cast<f32x4*>(po + hi_off + 4 * ce) = f32x4{hi[0], hi[1], hi[2], hi[3]};
    } else {
      const bool bf = a.q_dtype == MKV_DTYPE_BF16;
      auto pack = [&](float x, float y) -> uint32_t {
        const uint32_t bx = bf ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
        const uint32_t by = bf ? f32_to_bf16_bits(y) : f32_to_f16_bits(y);
        return bx | (by << 16);
      };
      uint16_t* po = reinterpret_cast<uint16_t*>(a.out) + o;
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      if (keep_lo) *reinterpret_cast<u32x2*>(po + 4 * ce) = u32x2{pack(lo[0], lo[1]), pack(lo[2], lo[3])};
      if (keep_hi)
        *reinterpret_cast<u32x2*>(po + hi_off + 4 * ce) = u32x2{pack(hi[0], hi[1]), pack(hi[2], hi[3])};
    }
  }
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

int tok_per_wg_for(int group) { return kRowsPerWg / group; }

int64_t tiles_upper_bound(int num_seqs, int64_t total_q, int group) {
  const int tpw = tok_per_wg_for(group);
  return (total_q + tpw - 1) / tpw + num_seqs;
}

template <int KV_DT, bool PAGED, bool QSPLIT>
int launch_prefill(const PrefillArgs& a, hipStream_t s) {
  const size_t lds = kTileListOffset + (a.inline_list ? sizeof(TilePick) : 0);
  int64_t nwg = a.tiles_ub * a.num_kv_heads;
  nwg = ((nwg + kXcds - 1) / kXcds) * kXcds;
  if (a.pair) {
    if constexpr (kPrefill2w<KV_DT, QSPLIT, true>)
      hipLaunchKernelGGL((prefill_mfma_2w_kernel<KV_DT, PAGED, QSPLIT, true>), dim3((unsigned)nwg),
                         dim3(kPfThreads), lds, s, a);
    else
      hipLaunchKernelGGL((prefill_mfma_kernel<KV_DT, PAGED, QSPLIT, true>), dim3((unsigned)nwg), dim3(kPfThreads),
                         lds, s, a);
  } else {
    if constexpr (kPrefill2w<KV_DT, QSPLIT, false>)
      hipLaunchKernelGGL((prefill_mfma_2w_kernel<KV_DT, PAGED, QSPLIT, false>), dim3((unsigned)nwg),
                         dim3(kPfThreads), lds, s, a);
    else
      hipLaunchKernelGGL((prefill_mfma_kernel<KV_DT, PAGED, QSPLIT, false>), dim3((unsigned)nwg), dim3(kPfThreads),
                         lds, s, a);
  }
  return (int)hipGetLastError();
}

template <bool PAGED>
int launch_prefill_f32(const PrefillArgs& a, hipStream_t s) {
  const size_t lds = kTileListOffset + (a.inline_list ? sizeof(TilePick) : 0);
  int64_t nwg = a.tiles_ub * a.num_kv_heads;
  nwg = ((nwg + kXcds - 1) / kXcds) * kXcds;
  if (a.pair)
    hipLaunchKernelGGL((prefill_f32_kernel<PAGED, true>), dim3((unsigned)nwg), dim3(kPfThreads), lds, s, a);
  else
    hipLaunchKernelGGL((prefill_f32_kernel<PAGED, false>), dim3((unsigned)nwg), dim3(kPfThreads), lds, s, a);
  return (int)hipGetLastError();
}

size_t prefill_ws_bytes(int num_seqs) { return ((size_t)(2 * num_seqs + 1) * sizeof(int32_t) + 255) / 256 * 256; }

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" size_t mkv_paged_prefill_workspace_size(int num_seqs, int64_t total_q, int num_heads,
                                                   int num_kv_heads) {
  (void)total_q;
  (void)num_heads;
  (void)num_kv_heads;
  return num_seqs > 0 ? prefill_ws_bytes(num_seqs) : 0;
}

extern "C" size_t mkv_flash_prefill_workspace_size(int num_seqs, int64_t total, int num_heads,
                                                   int num_kv_heads) {
  return mkv_paged_prefill_workspace_size(num_seqs, total, num_heads, num_kv_heads);
}

namespace {

// Shape checks shared by both entry points; fills the kernel's view of the
// heads (head_dim 64: KV heads read in pairs, kQDim in mkv_device.hpp).
int check_common(int num_seqs, int64_t total_q, int num_heads, int num_kv_heads, int head_dim,
                 int q_dtype, int kv_dtype, PrefillArgs& a) {
  if (num_seqs < 0 || total_q < 0 || num_heads <= 0 || num_kv_heads <= 0) return MKV_ERR_BAD_SHAPE;
  if (head_dim != kHeadDim && head_dim != kHeadDim / 2) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  if (num_heads % num_kv_heads) return MKV_ERR_UNSUPPORTED_GROUP;
  const int g = num_heads / num_kv_heads;
  const bool pair = head_dim == kHeadDim / 2;
  if (pair && (num_kv_heads & 1)) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  if (g < 1 || g > (pair ? 8 : 16)) return MKV_ERR_UNSUPPORTED_GROUP;
  a.num_heads = num_heads;
  a.num_kv_heads = pair ? num_kv_heads / 2 : num_kv_heads;
  a.group = pair ? 2 * g : g;
  a.scale_heads = num_kv_heads;
  a.pair = pair ? 1 : 0;
  if (q_dtype != MKV_DTYPE_F32 && q_dtype != MKV_DTYPE_BF16 && q_dtype != MKV_DTYPE_F16)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (kv_dtype != MKV_DTYPE_F32 && kv_dtype != MKV_DTYPE_BF16 && kv_dtype != MKV_DTYPE_F16 &&
      kv_dtype != MKV_DTYPE_FP8E4M3 && kv_dtype != MKV_DTYPE_I8)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  return MKV_OK;
}

template <bool PAGED>
int dispatch_prefill(PrefillArgs& a, int kv_dtype, void* workspace, size_t workspace_bytes,
                     hipStream_t s) {
  if (workspace_bytes < prefill_ws_bytes(a.num_seqs) || !workspace) return MKV_ERR_WORKSPACE_TOO_SMALL;
  a.tile_start = reinterpret_cast<int32_t*>(workspace);
  int32_t* order = a.tile_start + a.num_seqs + 1;
  a.order = order;
  a.tok_per_wg = tok_per_wg_for(a.group);
  a.tiles_ub = tiles_upper_bound(a.num_seqs, a.total_q, a.group);
  a.inline_list = a.num_seqs <= kInlineSeqs;
  if (!a.inline_list) {
    const int64_t ctx_cap = PAGED ? ((int64_t)a.idx.max_blocks << a.idx.bs_log2) : 0;
    hipLaunchKernelGGL(prefill_tile_scan_kernel, dim3(1), dim3(256), 0, s, a.cu_seqlens_q,
                       PAGED ? a.context_lens : nullptr, a.ctx_i64, ctx_cap, a.num_seqs, a.tok_per_wg,
                       a.tile_start, order);
  }
  // per-token-head caches run fp16 operands: a bf16 / fp16 q is exact in
  // fp16 after its power-of-two normalisation, an fp32 q takes two terms
  const bool q16 = a.q_dtype != MKV_DTYPE_F32;
  switch (kv_dtype) {
    case MKV_DTYPE_F32: return launch_prefill_f32<PAGED>(a, s);
    case MKV_DTYPE_FP8E4M3: return launch_prefill<MKV_DTYPE_FP8E4M3, PAGED, false>(a, s);
    case kKvFp8PerToken:
      if constexpr (PAGED)
        return q16 ? launch_prefill<kKvFp8PerToken, true, false>(a, s) : launch_prefill<kKvFp8PerToken, true, true>(a, s);
      return MKV_ERR_UNSUPPORTED_DTYPE;
    case kKvI8PerToken:
      if constexpr (PAGED)
        return q16 ? launch_prefill<kKvI8PerToken, true, false>(a, s) : launch_prefill<kKvI8PerToken, true, true>(a, s);
      return MKV_ERR_UNSUPPORTED_DTYPE;
    case MKV_DTYPE_BF16:
      return a.q_dtype == MKV_DTYPE_BF16 ? launch_prefill<MKV_DTYPE_BF16, PAGED, false>(a, s)
                                         : launch_prefill<MKV_DTYPE_BF16, PAGED, true>(a, s);
    default: return launch_prefill<MKV_DTYPE_F16, PAGED, false>(a, s);
  }
}

}  // namespace

extern "C" int mkv_paged_prefill(void* out, const void* q, int q_dtype, const void* k_cache,
                                 const void* v_cache, int kv_dtype, int64_t num_blocks,
                                 const float* k_scale, const float* v_scale, int kv_scale_mode,
                                 const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                 const void* context_lens, int context_lens_dtype,
                                 const int32_t* cu_seqlens_q, const int64_t* positions,
                                 int num_seqs, int64_t total_q, int num_heads, int num_kv_heads,
                                 int head_dim, int block_size, float sm_scale, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  PrefillArgs a{};
  int st = check_common(num_seqs, total_q, num_heads, num_kv_heads, head_dim, q_dtype, kv_dtype, a);
  if (st) return st;
  if (num_seqs == 0 || total_q == 0) return MKV_OK;
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens || !cu_seqlens_q ||
      !positions)
    return MKV_ERR_NULL_POINTER;
  // FP8: per-tensor or per-token-head scales; INT8: per-token-head only
  int fmt = kv_dtype;
  if (kv_scale_mode == MKV_SCALE_PER_TOKEN_HEAD && (kv_dtype == MKV_DTYPE_FP8E4M3 || kv_dtype == MKV_DTYPE_I8))
    fmt = kv_dtype == MKV_DTYPE_I8 ? kKvI8PerToken : kKvFp8PerToken;
  else if (kv_dtype == MKV_DTYPE_I8 || (kv_dtype == MKV_DTYPE_FP8E4M3 && kv_scale_mode != MKV_SCALE_PER_TENSOR))
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if ((kv_dtype == MKV_DTYPE_FP8E4M3 || kv_dtype == MKV_DTYPE_I8) && (!k_scale || !v_scale))
    return MKV_ERR_NULL_POINTER;
  if (context_lens_dtype != MKV_INDEX_I32 && context_lens_dtype != MKV_INDEX_I64)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 4) return MKV_ERR_BAD_BLOCK_SIZE;
  if (bt_stride < max_blocks || max_blocks < 0 || num_blocks < 0) return MKV_ERR_BAD_STRIDE;
  // token slots of the pool are indexed in 32 bits (a pool of 2^32 slots is
  // 512 GiB per cache at one byte per element and head_dim 128)
  if (num_blocks > ((int64_t)1 << (32 - bs_log2))) return MKV_ERR_BAD_SHAPE;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u)
    return MKV_ERR_MISALIGNED;
  a.out = out;
  a.q = q;
  a.q_dtype = q_dtype;
  a.k = reinterpret_cast<const char*>(k_cache);
  a.v = reinterpret_cast<const char*>(v_cache);
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.idx.block_tables = block_tables;
  a.idx.bt_stride = bt_stride;
  a.idx.max_blocks = max_blocks;
  a.idx.num_blocks = num_blocks;
  a.idx.bs_log2 = bs_log2;
  a.idx.row_elems = (int64_t)num_kv_heads * head_dim;
  a.context_lens = context_lens;
  a.ctx_i64 = context_lens_dtype == MKV_INDEX_I64;
  a.cu_seqlens_q = cu_seqlens_q;
  a.positions = positions;
  a.num_seqs = num_seqs;
  a.total_q = total_q;
  a.sm_scale = sm_scale;
  return dispatch_prefill<true>(a, fmt, workspace, workspace_bytes,
                                reinterpret_cast<hipStream_t>(stream));
}

extern "C" int mkv_flash_prefill(void* out, const void* q, const void* k, const void* v, int dtype,
                                 const int32_t* cu_seqlens, int num_seqs, int64_t total,
                                 int num_heads, int num_kv_heads, int head_dim, float sm_scale,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  PrefillArgs a{};
  int st = check_common(num_seqs, total, num_heads, num_kv_heads, head_dim, dtype, dtype, a);
  if (st) return st;
  if (num_seqs == 0 || total == 0) return MKV_OK;
  if (!out || !q || !k || !v || !cu_seqlens) return MKV_ERR_NULL_POINTER;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u)
    return MKV_ERR_MISALIGNED;
  a.out = out;
  a.q = q;
  a.q_dtype = dtype;
  a.k = reinterpret_cast<const char*>(k);
  a.v = reinterpret_cast<const char*>(v);
  a.cu_seqlens_q = cu_seqlens;
  a.num_seqs = num_seqs;
  a.total_q = total;
  a.sm_scale = sm_scale;
  return dispatch_prefill<false>(a, dtype, workspace, workspace_bytes,
                                 reinterpret_cast<hipStream_t>(stream));
}
