// K2: paged decode attention for gfx950.
//
// Reference semantics: paged_attention_decode (attention.py:895-950, kernel
// :517-646) and paged_attention_decode_quantized (attention.py:1213-1268):
// per-tensor FP8 (kernel :953-1121, dequant :1051-1062/:1098-1107) and
// per-token-head FP8 / INT8 (tile kernel :1124-1210).
//
// Work item = (sequence b, kv head g, split s): one wavefront reads the
// split's K/V tokens of kv head g exactly once and serves all G = Hq/Hkv
// query heads of the group (the reference launches one program per query
// head and so reads K/V G times).
//
// Per 32-token tile the wave computes S^T = K q^T and O += P V on the MFMA
// units with operands loaded straight from HBM into registers:
//   * QK: A = K (16 tokens x 32 dims per lane group), B = q^T (dims x heads).
//     The contraction order over head_dim is a free permutation, so each lane
//     loads 32 *contiguous* dims of one token row.
//   * PV: A = P (heads x tokens), B = V (tokens x dims).  The token set of a
//     lane group is chosen to be exactly the 8 tokens whose scores that lane
//     already holds in its QK accumulators, so P never leaves registers; the
//     output-dim order is also free, so each lane loads 8 contiguous dims of
//     8 token rows and transposes them with v_perm (bytes for FP8,
//     half-words for 16-bit caches).
//   * FP8 bytes convert exactly to fp16 (v_cvt_scalef32_pk_f16_fp8) and run
//     on the fp16 MFMA; q is normalised by a power of two so it is exact in
//     fp16, and the per-tensor k/v scales are applied to scores / output in
//     fp32 (legal because the scale is per tensor).
//   * Per-token-head FP8 / INT8 codes convert exactly to bf16 and run on the
//     bf16 MFMA.  Each lane loads one scale per tile (K or V scale of one of
//     the 8 tokens its 16-lane row holds scores for) and DPP row broadcasts
//     hand every lane the 16 it needs: the K scale multiplies the score, the
//     V scale folds into P (P * v_scale, split into two bf16 terms), and the
//     softmax denominator sums the unscaled P, as the reference does.
// Splits that do not cover a whole sequence write (acc, m, l) partials that a
// second kernel merges with the log-sum-exp rule.
#include <mutex>

#include "mkv_device.hpp"
#include "qkv_producer.hpp"

namespace mkv {
namespace {

constexpr int kHeadDim = 128;
constexpr int kDecWaves = 4;
constexpr float kNegBig = -1e30f;

struct DecodeArgs {
  void* out;
  int64_t out_stride;
  const void* q;
  int64_t q_stride;
  int q_dtype;
  const char* k_cache;
  const char* v_cache;
  const float* k_scale;  // per tensor: one fp32; per token head: (slots, Hkv)
  const float* v_scale;
  PagedIndex idx;
  const void* context_lens;
  int ctx_i64;
  int batch;
  int num_heads;
  int num_kv_heads;
  int group;
  float sm_scale;
  int split_tokens;
  int max_splits;
  float* ws_acc;  // [batch * num_heads][max_splits][head_dim]
  float* ws_ml;   // [batch * num_heads][max_splits][2]  (m, l), log2 domain
  // stream-K decomposition (16-bit KV): partial slots per wave and metadata
  int* sk_meta;     // [batch + 1] tile prefix per sequence, then [batch] x 3 merge
                    // metadata (first / last contributing group, slot of the first)
  int seq_cost;     // split cost of entering a sequence, in quarter columns
  int defer;        // finishes a stream-K wave may hold in LDS until its range ends
  int first_pct;    // percent of the split that the first dispatch round's groups take
  int num_waves;    // persistent waves in the grid
  int first_waves;  // waves of the first dispatch round (== num_waves: even split)
  int scale_heads;  // KV heads of the per-token-head scale tensors (the caller's Hkv)
  int pair;         // head_dim 64: KV heads read in pairs (kQDim in mkv_device.hpp)
};

MKV_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Store 8 consecutive fp32 values in the output dtype.
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
      const uint32_t hi =
          dt == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
      a[j] = lo | (hi << 16);
    }
    st16(reinterpret_cast<uint16_t*>(out) + off, a);
  }
}

struct WorkItem {
  int b, kvh, split, num_splits;
  int t_begin, t_end;  // token range of this split (context lengths fit in 31 bits)
};

// Decode the flat work index; returns false if the item has nothing to do.
// A sequence with context length 0 keeps split 0 so that zeros get written.
// w must be wave-uniform so that everything derived from it stays scalar.
MKV_DEV bool decode_work_item(const DecodeArgs& a, int64_t w, WorkItem& it) {
  const int64_t per_split = (int64_t)a.batch * a.num_kv_heads;
  if (w >= per_split * a.max_splits) return false;
  it.split = (int)(w / per_split);
  const int64_t rem = w - (int64_t)it.split * per_split;
  it.b = (int)(rem / a.num_kv_heads);
  it.kvh = (int)(rem - (int64_t)it.b * a.num_kv_heads);
  int64_t L = load_index(a.context_lens, it.b, a.ctx_i64);
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  it.num_splits = L > 0 ? (int)((L + a.split_tokens - 1) / a.split_tokens) : 1;
  if (it.split >= it.num_splits) return false;
  it.t_begin = it.split * a.split_tokens;
  it.t_end = (int)(it.t_begin + a.split_tokens < L ? it.t_begin + a.split_tokens : L);
  return true;
}

MKV_DEV int64_t wave_work_index() {
  return (int64_t)blockIdx.x * kDecWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Final normalisation / partial write for one wave.  Lane (kg, c) holds
// O[head 4kg + r][dim 8c + mm] in acc[mm][r]; m_col / l_col hold the running
// max and the (lane-group summed) denominator of head c.
template <bool PAIR>
MKV_DEV void finish_item(const DecodeArgs& a, const WorkItem& it, f32x4 (&acc)[8], float m_col,
                         float l_col, float v_mul) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * kg + r;
    const float lh = __shfl(l_col, h);
    const float mh = __shfl(m_col, h);
    if (h >= a.group) continue;
    const int hq = it.kvh * a.group + h;
    float x[8];
    if (it.num_splits == 1) {
      const float inv = lh > 0.0f ? v_mul / lh : 0.0f;
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) x[mm] = acc[mm][r] * inv;
      int col0;
      if (out_cols<PAIR>(a.group, h, c, col0))
        store_out8(a.out, a.q_dtype, (int64_t)it.b * a.out_stride + (int64_t)hq * kQDim<PAIR> + col0, x);
    } else {
      const int64_t slot = ((int64_t)it.b * a.num_heads + hq) * a.max_splits + it.split;
      float* p = a.ws_acc + slot * kHeadDim + 8 * c;
      u32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = __float_as_uint(acc[j][r]);
        hi[j] = __float_as_uint(acc[4 + j][r]);
      }
      st16(p, lo);
      st16(p + 4, hi);
      if (c == 0) {
        a.ws_ml[slot * 2] = mh;
        a.ws_ml[slot * 2 + 1] = lh;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit MFMA kernel: KV in FP8 (via exact fp16), bf16 or fp16.
// ---------------------------------------------------------------------------
// Raw-buffer descriptor word 3 for gfx9-class targets (untyped 32-bit data).
constexpr int kRsrcFlags = 0x00020000;
// A per-lane buffer offset beyond every descriptor's range: the load returns 0.
constexpr uint32_t kOob = 0x80000000u;
// Cache policy of the K/V loads.  The non-temporal hint (bit 1) speeds up
// streamed-once reads only when every load instruction covers whole 128-byte
// lines; when two instructions share a line it costs bandwidth instead.  The
// V loads and the FP8 K loads cover whole lines; the 16-bit K loads do not.
constexpr int kAuxNt = 2;
template <int KV_DT>
struct LoadPolicy {
  static constexpr int kK = DTypeInfo<KV_DT>::kBytes == 1 ? kAuxNt : 0;
  static constexpr int kV = kAuxNt;
};

// FP8 K rows are 128 bytes and an MFMA row is owned by the four lanes c +
// 16*kg, which keep bytes 32kg .. 32kg+31.  One load instruction can cover
// whole lines only if eight lanes read each row, so a 16-row sub-tile is read
// by two instructions: A reads rows 0-7 (lane c < 8: row c, bytes 32kg..+15;
// lane c >= 8: row c-8, bytes 32kg+16..+31), B reads rows 8-15 the other way
// round.  k_exchange() then swaps the borrowed halves between lanes c and
// c^8 (same kg) with one DPP rotate, leaving lane (c, kg) with bytes
// 32kg .. 32kg+15 of row c in piece 0 and 32kg+16 .. 32kg+31 in piece 1.
struct Fp8KLanes {
  int off_a, off_b;  // byte offsets inside the sub-tile (row * row_bytes + col)
  int row_a, row_b;  // rows the lane reads in instructions A and B
};
MKV_DEV Fp8KLanes fp8_k_lanes(int row_bytes) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  const bool top = c < 8;
  Fp8KLanes f;
  f.row_a = c & 7;
  f.row_b = (c & 7) + 8;
  f.off_a = f.row_a * row_bytes + 32 * kg + (top ? 0 : 16);
  f.off_b = f.row_b * row_bytes + 32 * kg + (top ? 16 : 0);
  return f;
}
MKV_DEV void k_exchange(u32x4& a, u32x4& b) {
  const bool top = (threadIdx.x & 15) < 8;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t send = top ? b[d] : a[d];
    const uint32_t own = top ? a[d] : b[d];
    // row_ror:8 inside each 16-lane row: lane c receives from lane c ^ 8
    b[d] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send, 0x128, 0xf, 0xf, false);
    a[d] = own;
  }
}

// Descriptor over the rows of one block that start at `row` (token offset in
// the block) for one KV head: [base, end of block).  An absent block (phys <
// 0) gets an empty range, so every load through it returns zeros.  All inputs
// are wave-uniform.
MKV_DEV __amdgpu_buffer_rsrc_t rows_rsrc(const char* pool, int64_t phys, int64_t blk_bytes,
                                        int64_t off_in_blk) {
  // selects, not branches: a branch here would split the load sequence and
  // make the wait-count pass drain the prefetch at the join
  const bool ok = phys >= 0;
  const char* base = pool + (ok ? phys * blk_bytes + off_in_blk : 0);
  const int num = ok ? (int)(blk_bytes - off_in_blk) : 0;
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, num, kRsrcFlags);
}

// Per work item constants of the tile loads.
struct ItemLoad {
  int k_voff;    // lane byte offset of its K row chunk inside a 16-token group
  int v_voff;    // lane byte offset of its V row chunk (token 4kg, dims 8c..)
  int row_bytes; // bytes per token row (all KV heads)
  int64_t blk_bytes;
  int64_t head_bytes;  // byte offset of this KV head inside a token row
};

template <int KV_DT>
MKV_DEV ItemLoad item_load_setup(const DecodeArgs& a, const WorkItem& it) {
  constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  ItemLoad L;
  L.row_bytes = (int)(a.idx.row_elems * kEb);
  L.blk_bytes = (int64_t)L.row_bytes << a.idx.bs_log2;
  L.head_bytes = (int64_t)it.kvh * kHeadDim * kEb;
  L.k_voff = c * L.row_bytes + 32 * kg * kEb;
  L.v_voff = 4 * kg * L.row_bytes + 8 * c * kEb;
  return L;
}

struct PhysPair {
  int64_t p[2];
};

// Block-table entries of the 16-token halves at t0 and t0 + 16 of sequence
// b (-1 at or past t_end, or absent).  Wave-uniform lookups through the
// constant address space, i.e. scalar loads counted on lgkmcnt: the split-K
// and workgroup loops issue them one tile ahead of the K/V loads that use
// them, so no lookup waits for the tiles in flight, and a range may span any
// number of blocks.
MKV_DEV int64_t item_phys1(const DecodeArgs& a, int b, int tok, int t_end) {
  return tok < t_end ? a.idx.physical_block(b, tok >> a.idx.bs_log2) : -1;
}
MKV_DEV PhysPair item_phys(const DecodeArgs& a, int b, int t0, int t_end) {
  PhysPair ph;
#pragma unroll
  for (int h = 0; h < 2; ++h) ph.p[h] = item_phys1(a, b, t0 + 16 * h, t_end);
  return ph;
}

template <int KV_DT>
struct Tile16 {
  // K: 2 sub-tiles of 16 tokens x 32 dims per lane; V: 8 tokens x 8 dims.
  static constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  static constexpr int kKVec = (32 * kEb) / 16;  // 16-byte loads per K row chunk
  using VT = typename std::conditional<kEb == 1, u32x2, u32x4>::type;
  u32x4 k[2][kKVec];
  VT v[8];
  float sc;    // per-token-head formats: one K or V scale (load_tile_scales)
  float sc2;   // with head pairing: the same scale of the pair's second KV head
  bool ok[2];  // sub-tile block present
};

// Per-token-head scales of the 32-token tile at t0 of KV head kvh (block
// entries ph0 / ph1 of its two 16-token halves).  Lane (c, kg) loads the K
// (c < 8) or V (c >= 8) scale of token t0 + 16m + 4kg + r with m = (c >> 2) & 1,
// r = c & 3: row kg of the wave then holds exactly the 16 scales of the 8
// tokens whose scores it computes.  With head pairing the lane also loads
// the scale of the pair's second KV head (the next entry).  An absent block
// reads slot 0 of block 0 (a valid address; the value is masked where it is
// used).  The loads are issued unconditionally, like the K/V loads.
typedef const float __attribute__((address_space(1))) global_f32;
template <int KV_DT, bool PAIR>
MKV_DEV void load_tile_scales(const DecodeArgs& a, int64_t ph0, int64_t ph1, int t0, int kvh,
                              Tile16<KV_DT>& T) {
  if constexpr (kPerTokenScale<KV_DT>) {
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, kg = lane >> 4;
    const int bs_mask = (1 << a.idx.bs_log2) - 1;
    const int sh = a.scale_heads;
    const int kvr = PAIR ? 2 * kvh : kvh;  // the caller's KV head
    // scale index of the first token of each half (the host checks that the
    // scale tensor has fewer than 2^31 entries)
    const int s0 = (int)((((ph0 < 0 ? 0 : ph0) << a.idx.bs_log2) + (t0 & bs_mask)) * sh) + kvr;
    const int s1 = (int)((((ph1 < 0 ? 0 : ph1) << a.idx.bs_log2) + ((t0 + 16) & bs_mask)) * sh) + kvr;
    const int idx = ((c & 4) ? s1 : s0) + (4 * kg + (c & 3)) * sh;
    const float* base = c < 8 ? a.k_scale : a.v_scale;
    T.sc = *((global_f32*)(base + idx));
    if constexpr (PAIR) T.sc2 = *((global_f32*)(base + idx + 1));
  }
}

// Issue the K/V loads of one 32-token tile through the per-half descriptors
// rk/rv (rows t0 .. t0+15 and t0+16 .. t0+31).  Rows at or past t_end read as
// zeros (out-of-range offset); no branches.
template <int KV_DT>
MKV_DEV void load_tile_rows(const __amdgpu_buffer_rsrc_t (&rk)[2], const __amdgpu_buffer_rsrc_t (&rv)[2],
                            int t0, int t_end, int k_voff, int v_voff, int row_bytes, Tile16<KV_DT>& T) {
  constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  if constexpr (kEb == 1) {
    const Fp8KLanes f = fp8_k_lanes(row_bytes);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t oa = (t0 + 16 * m + f.row_a < t_end) ? (uint32_t)f.off_a : kOob;
      const uint32_t ob = (t0 + 16 * m + f.row_b < t_end) ? (uint32_t)f.off_b : kOob;
      T.k[m][0] = __builtin_amdgcn_raw_buffer_load_b128(rk[m], oa, 0, LoadPolicy<KV_DT>::kK);
      T.k[m][1] = __builtin_amdgcn_raw_buffer_load_b128(rk[m], ob, 0, LoadPolicy<KV_DT>::kK);
    }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t off = (t0 + 16 * m + c < t_end) ? (uint32_t)k_voff : kOob;
#pragma unroll
      for (int i = 0; i < Tile16<KV_DT>::kKVec; ++i)
        T.k[m][i] = __builtin_amdgcn_raw_buffer_load_b128(rk[m], off + 16 * i, 0, LoadPolicy<KV_DT>::kK);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int hf = i >> 2, r = i & 3;
    const uint32_t off =
        (t0 + 16 * hf + 4 * kg + r < t_end) ? (uint32_t)(v_voff + r * row_bytes) : kOob;
    if constexpr (kEb == 1)
      T.v[i] = __builtin_amdgcn_raw_buffer_load_b64(rv[hf], off, 0, LoadPolicy<KV_DT>::kV);
    else
      T.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv[hf], off, 0, LoadPolicy<KV_DT>::kV);
  }
}

// Issue every load of the 32-token tile starting at t0 (wave-uniform) with
// its block-table entries ph (item_phys).  Tokens past the split end and
// absent blocks read as zeros; no branches.
template <int KV_DT, bool PAIR>
MKV_DEV void load_tile16(const DecodeArgs& a, const WorkItem& it, const ItemLoad& L, int t0,
                         const PhysPair& ph, Tile16<KV_DT>& T) {
  const int bs_mask = (1 << a.idx.bs_log2) - 1;
  __amdgpu_buffer_rsrc_t rk[2], rv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t off = L.head_bytes + (int64_t)((t0 + 16 * h) & bs_mask) * L.row_bytes;
    rk[h] = rows_rsrc(a.k_cache, ph.p[h], L.blk_bytes, off);
    rv[h] = rows_rsrc(a.v_cache, ph.p[h], L.blk_bytes, off);
    T.ok[h] = ph.p[h] >= 0;
  }
  load_tile_rows<KV_DT>(rk, rv, t0, it.t_end, L.k_voff, L.v_voff, L.row_bytes, T);
  load_tile_scales<KV_DT, PAIR>(a, ph.p[0], ph.p[1], t0, it.kvh, T);
}

// Formats that run on the bf16 MFMA (bf16 caches and the per-token-head codes,
// which convert to bf16 exactly); the others run on the fp16 MFMA.
template <int KV_DT>
constexpr bool kBf16Mfma = KV_DT == MKV_DTYPE_BF16 || kPerTokenScale<KV_DT>;

template <int KV_DT>
using Op16 = typename std::conditional<kBf16Mfma<KV_DT>, bf16x8, f16x8>::type;

template <int KV_DT>
MKV_DEV f32x4 mfma16(Op16<KV_DT> A, Op16<KV_DT> B, f32x4 C) {
  if constexpr (kBf16Mfma<KV_DT>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B, C, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, C, 0, 0, 0);
}

// Four fp32 -> MFMA operand element type.
template <int KV_DT>
MKV_DEV Op16<KV_DT> to_op16(const float* x) {
  Op16<KV_DT> r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (kBf16Mfma<KV_DT>)
      r[j] = (__bf16)x[j];
    else
      r[j] = (_Float16)x[j];
  }
  return r;
}

// Eight 1-byte per-token-head codes (d0 bytes 0-3, d1 bytes 0-3) -> bf16.
template <int KV_DT>
MKV_DEV bf16x8 bytes8_to_bf16x8(uint32_t d0, uint32_t d1) {
  bf16x2 a0, a1, a2, a3;
  if constexpr (KV_DT == kKvFp8PerToken) {
    a0 = fp8x2_to_bf16x2<false>(d0), a1 = fp8x2_to_bf16x2<true>(d0);
    a2 = fp8x2_to_bf16x2<false>(d1), a3 = fp8x2_to_bf16x2<true>(d1);
  } else {
    a0 = i8x2_to_bf16x2<false>(d0), a1 = i8x2_to_bf16x2<true>(d0);
    a2 = i8x2_to_bf16x2<false>(d1), a3 = i8x2_to_bf16x2<true>(d1);
  }
  return bf16x8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
}

// A operand of QK step st for K sub-tile m (8 dims: 32kg + 8st .. +7) from
// the lane's K words (FP8 words already passed through k_exchange).
template <int KV_DT>
MKV_DEV Op16<KV_DT> k_operand(const u32x4 (&K)[2][Tile16<KV_DT>::kKVec], int m, int st) {
  if constexpr (KV_DT == MKV_DTYPE_FP8E4M3) {
    const u32x4 w = K[m][st >> 1];
    const uint32_t d0 = (st & 1) ? w[2] : w[0];
    const uint32_t d1 = (st & 1) ? w[3] : w[1];
    const f16x2 a0 = fp8x2_to_f16x2<false>(d0), a1 = fp8x2_to_f16x2<true>(d0);
    const f16x2 a2 = fp8x2_to_f16x2<false>(d1), a3 = fp8x2_to_f16x2<true>(d1);
    return f16x8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  } else if constexpr (kPerTokenScale<KV_DT>) {
    const u32x4 w = K[m][st >> 1];
    const uint32_t d0 = (st & 1) ? w[2] : w[0];
    const uint32_t d1 = (st & 1) ? w[3] : w[1];
    return bytes8_to_bf16x8<KV_DT>(d0, d1);
  } else {
    return __builtin_bit_cast(Op16<KV_DT>, K[m][st]);
  }
}

// B operands of the 8 PV MFMAs (one per output dim 8c + mm): element j is
// V[token T_j][8c + mm].
template <int KV_DT>
MKV_DEV void v_operands(const Tile16<KV_DT>& T, Op16<KV_DT> (&B)[8]) {
  if constexpr (DTypeInfo<KV_DT>::kBytes == 1) {
    uint32_t X[8], Y[8];
    transpose_bytes_4x4(T.v[0][0], T.v[1][0], T.v[2][0], T.v[3][0], X[0], X[1], X[2], X[3]);
    transpose_bytes_4x4(T.v[0][1], T.v[1][1], T.v[2][1], T.v[3][1], X[4], X[5], X[6], X[7]);
    transpose_bytes_4x4(T.v[4][0], T.v[5][0], T.v[6][0], T.v[7][0], Y[0], Y[1], Y[2], Y[3]);
    transpose_bytes_4x4(T.v[4][1], T.v[5][1], T.v[6][1], T.v[7][1], Y[4], Y[5], Y[6], Y[7]);
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) {
      if constexpr (kPerTokenScale<KV_DT>) {
        B[mm] = bytes8_to_bf16x8<KV_DT>(X[mm], Y[mm]);
      } else {
        const f16x2 a0 = fp8x2_to_f16x2<false>(X[mm]), a1 = fp8x2_to_f16x2<true>(X[mm]);
        const f16x2 a2 = fp8x2_to_f16x2<false>(Y[mm]), a3 = fp8x2_to_f16x2<true>(Y[mm]);
        B[mm] = f16x8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      u32x4 lo, hi;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        lo[q] = pack_lo16(T.v[2 * q][p], T.v[2 * q + 1][p]);
        hi[q] = pack_hi16(T.v[2 * q][p], T.v[2 * q + 1][p]);
      }
      B[2 * p] = __builtin_bit_cast(Op16<KV_DT>, lo);
      B[2 * p + 1] = __builtin_bit_cast(Op16<KV_DT>, hi);
    }
  }
}

// q as MFMA operands (dims 32kg + 8st .. +7 of head c in hi[st]).  A bf16
// MFMA format holds an fp32 or fp16 q only to 8 bits:
// then lo[st] carries the rounding residual and each QK step takes a second
// MFMA (split), giving ~16 significant bits like the fp32 reference.
template <int KV_DT>
struct QOps {
  Op16<KV_DT> hi[4];
  Op16<KV_DT> lo[4];
  bool split;
};

// The 16 scales that row kg of the wave loaded (load_tile_scales): K scales
// of its tokens 4m + r from lanes 0-7, V scales from lanes 8-15.
MKV_DEV void row_scales(float sc, float (&ks)[8], float (&vs)[8]) {
  ks[0] = row_bcast<0>(sc), ks[1] = row_bcast<1>(sc), ks[2] = row_bcast<2>(sc);
  ks[3] = row_bcast<3>(sc), ks[4] = row_bcast<4>(sc), ks[5] = row_bcast<5>(sc);
  ks[6] = row_bcast<6>(sc), ks[7] = row_bcast<7>(sc);
  vs[0] = row_bcast<8>(sc), vs[1] = row_bcast<9>(sc), vs[2] = row_bcast<10>(sc);
  vs[3] = row_bcast<11>(sc), vs[4] = row_bcast<12>(sc), vs[5] = row_bcast<13>(sc);
  vs[6] = row_bcast<14>(sc), vs[7] = row_bcast<15>(sc);
}

// One 32-token tile: S^T = K q^T, online softmax (log2 domain), O += P V.
// t0: first token of the tile, t_end: end of the visible range.  hi (head
// pairing, per-token-head formats): this lane's head c belongs to the
// pair's second KV head, whose scales it uses.
template <int KV_DT, bool PAIR>
MKV_DEV void compute_tile16(const Tile16<KV_DT>& cur, int t0, int t_end, const QOps<KV_DT>& qop,
                            float score_mul, f32x4 (&acc)[8], float& m_run, float& l_run, bool hi) {
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4;
  // S^T = K q^T: lane holds scores of tokens t0 + 16m + 4kg + r for head c.
  u32x4 kw[2][Tile16<KV_DT>::kKVec];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int i = 0; i < Tile16<KV_DT>::kKVec; ++i) kw[m][i] = cur.k[m][i];
    if constexpr (DTypeInfo<KV_DT>::kBytes == 1) k_exchange(kw[m][0], kw[m][1]);
  }
  f32x4 s[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    s[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const Op16<KV_DT> kop = k_operand<KV_DT>(kw, m, st);
      s[m] = mfma16<KV_DT>(kop, qop.hi[st], s[m]);
      if constexpr (kBf16Mfma<KV_DT>)
        if (qop.split) s[m] = mfma16<KV_DT>(kop, qop.lo[st], s[m]);
    }
  }
  // Per-token-head formats: K scales (lanes 0-7 of the row) and V scales
  // (lanes 8-15) of this lane's tokens 16m + 4kg + r, index 4m + r.
  float ks[8], vs[8];
  if constexpr (kPerTokenScale<KV_DT>) {
    row_scales(cur.sc, ks, vs);
    if constexpr (PAIR) {
      float ks2[8], vs2[8];
      row_scales(cur.sc2, ks2, vs2);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ks[j] = hi ? ks2[j] : ks[j];
        vs[j] = hi ? vs2[j] : vs[j];
      }
    }
  }
  float mx = kNegBig;
  bool okt[8];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = t0 + 16 * m + 4 * kg + r < t_end && cur.ok[m];
      okt[4 * m + r] = ok;
      float sv = s[m][r] * score_mul;
      if constexpr (kPerTokenScale<KV_DT>) sv *= ks[4 * m + r];
      s[m][r] = ok ? sv : -__builtin_huge_valf();
      mx = fmaxf(mx, s[m][r]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m_run, mx);
  const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
  m_run = m_new;
  float p[8];
  float psum = 0.0f;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[4 * m + r] = __builtin_amdgcn_exp2f(s[m][r] - m_new);
      psum += p[4 * m + r];
    }
  }
  l_run = l_run * alpha + psum;
  // Rescale the output accumulators of heads 4kg + r.
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * kg + r);
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) acc[mm][r] *= ar;
    }
  }
  // PV weights: P, or P * v_scale of the token for per-token-head formats
  // (zero for masked tokens, whatever scale the masked slot holds).
  float pw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (kPerTokenScale<KV_DT>)
      pw[j] = okt[j] ? p[j] * vs[j] : 0.0f;
    else
      pw[j] = p[j];
  }
  const Op16<KV_DT> pop = to_op16<KV_DT>(pw);
  Op16<KV_DT> vop[8];
  v_operands<KV_DT>(cur, vop);
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = mfma16<KV_DT>(pop, vop[mm], acc[mm]);
  if constexpr (kBf16Mfma<KV_DT>) {
    // bf16 keeps 8 significant bits of the weights; add the rounding residual
    // as a second bf16 term so they carry ~16 bits like the fp32 reference.
    float plo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) plo[j] = pw[j] - (float)pop[j];
    const Op16<KV_DT> plop = to_op16<KV_DT>(plo);
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) acc[mm] = mfma16<KV_DT>(plop, vop[mm], acc[mm]);
  }
}

// MFMA operands of q (the lane holds dims 32kg .. 32kg+31 of head c of the
// group, zero for padding heads); returns the fp32 factor that maps MFMA
// scores to the log2-domain logits.  fp16 operands are normalised by a power
// of two so q is exact and in range; k_scale (per-tensor FP8) and
// sm_scale*log2(e) stay in fp32.
template <int KV_DT>
MKV_DEV float q_operands(const DecodeArgs& a, float (&qf)[32], QOps<KV_DT>& qop, float k_mul) {
  float score_mul = a.sm_scale * kLog2e * k_mul;
  if constexpr (!kBf16Mfma<KV_DT>) {
    float qm = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) qm = fmaxf(qm, fabsf(qf[i]));
    qm = wave_max(qm);
    if (qm > 0.0f && qm < __builtin_huge_valf()) {
      const int e = ilogbf(qm);
      const float f = ldexpf(1.0f, 8 - e);
#pragma unroll
      for (int i = 0; i < 32; ++i) qf[i] *= f;
      score_mul *= ldexpf(1.0f, e - 8);
    }
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) qop.hi[st] = to_op16<KV_DT>(qf + 8 * st);
  qop.split = false;
  if constexpr (kBf16Mfma<KV_DT>) {
    qop.split = a.q_dtype != MKV_DTYPE_BF16;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float r[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = qf[8 * st + j] - (float)qop.hi[st][j];
      qop.lo[st] = to_op16<KV_DT>(r);
    }
  }
  return score_mul;
}

// q of item (b, kvh) loaded and converted on the spot (any q dtype).  k_mul:
// the K dequantisation scale (1 for 16-bit caches).
template <int KV_DT, bool PAIR>
MKV_DEV float load_q_operands(const DecodeArgs& a, int b, int kvh, QOps<KV_DT>& qop, float k_mul) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  float qf[32];
  int d0;
  if (q_slice<PAIR>(a.group, c, kg, d0)) {
    const int64_t qoff = (int64_t)b * a.q_stride + (int64_t)(kvh * a.group + c) * kQDim<PAIR> + d0;
    load_q32(a.q, a.q_dtype, qoff, qf);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) qf[i] = 0.0f;
  }
  return q_operands<KV_DT>(a, qf, qop, k_mul);
}

// Raw 16-bit q of one item (dims 32kg .. 32kg+31 of head c), loaded a
// pipeline step before the item's first tile is computed so that its latency
// hides behind that tile's loads.
struct QStage {
  u32x4 w[4];
};

// Issue the q loads of item (b, kvh) for a bf16/fp16 q; padding heads read
// zeros.  With need == false the same four loads are issued with an empty
// range (nothing is read), so the stream of memory instructions is the same on
// every pipeline step: a load issued on only some steps makes the wait-count
// pass assume the worst at the join and wait for it, i.e. for a full memory
// round trip, before the next tile.
template <bool PAIR>
MKV_DEV void load_q_stage(const DecodeArgs& a, int b, int kvh, bool need, QStage& qs) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  constexpr int kQd = kQDim<PAIR>;
  const char* base = reinterpret_cast<const char*>(a.q) +
                     ((int64_t)b * a.q_stride + (int64_t)kvh * a.group * kQd) * 2;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      (void*)base, (short)0, need ? a.group * kQd * 2 : 0, kRsrcFlags);
  int d0;
  const uint32_t off = q_slice<PAIR>(a.group, c, kg, d0) ? (uint32_t)((c * kQd + d0) * 2) : kOob;
#pragma unroll
  for (int i = 0; i < 4; ++i) qs.w[i] = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
}

template <int KV_DT>
MKV_DEV float staged_q_operands(const DecodeArgs& a, const QStage& qs, QOps<KV_DT>& qop, float k_mul) {
  float qf[32];
  const bool bf = a.q_dtype == MKV_DTYPE_BF16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = qs.w[i][j];
      qf[8 * i + 2 * j] = bf ? bf16_bits_to_f32(w & 0xffffu) : f16_bits_to_f32(w & 0xffffu);
      qf[8 * i + 2 * j + 1] = bf ? bf16_bits_to_f32(w >> 16) : f16_bits_to_f32(w >> 16);
    }
  }
  return q_operands<KV_DT>(a, qf, qop, k_mul);
}

template <int KV_DT, bool PAIR>
MKV_DEV void split_decode(const DecodeArgs& a) {
  WorkItem it;
  if (!decode_work_item(a, wave_work_index(), it)) return;
  QOps<KV_DT> qop;
  const float k_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.k_scale) : 1.0f;
  const float score_mul = load_q_operands<KV_DT, PAIR>(a, it.b, it.kvh, qop, k_mul);
  const bool hi = PAIR && (threadIdx.x & 15) >= (a.group >> 1);

  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;


  // Software pipeline over two register tiles: the loads of tile i+1 are in
  // flight while tile i is computed, and the block-table entries of tile i+2
  // (scalar loads) while tile i+1's loads go out.  The prefetch is
  // unconditional (a tile past the split end reads zeros through the
  // descriptor range check and touches no memory), so no branch splits the
  // load stream and the waits before tile i only cover tile i's loads.
  if (it.t_begin < it.t_end) {
    const ItemLoad L = item_load_setup<KV_DT>(a, it);
    Tile16<KV_DT> ta, tb;
    load_tile16<KV_DT, PAIR>(a, it, L, it.t_begin, item_phys(a, it.b, it.t_begin, it.t_end), ta);
    PhysPair ph = item_phys(a, it.b, it.t_begin + 32, it.t_end);
    for (int t0 = it.t_begin;;) {
      load_tile16<KV_DT, PAIR>(a, it, L, t0 + 32, ph, tb);
      ph = item_phys(a, it.b, t0 + 64, it.t_end);
      compute_tile16<KV_DT, PAIR>(ta, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += 32;
      if (t0 >= it.t_end) break;
      load_tile16<KV_DT, PAIR>(a, it, L, t0 + 32, ph, ta);
      ph = item_phys(a, it.b, t0 + 64, it.t_end);
      compute_tile16<KV_DT, PAIR>(tb, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += 32;
      if (t0 >= it.t_end) break;
    }
  }
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  const float v_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.v_scale) : 1.0f;
  finish_item<PAIR>(a, it, acc, m_run, l_col, v_mul);
}

template <int KV_DT, bool PAIR>
__global__ __launch_bounds__(kDecWaves* kWave) void paged_decode_mfma16_kernel(DecodeArgs a) {
  split_decode<KV_DT, PAIR>(a);
}

// Per-token-head formats: two waves per SIMD requested explicitly (as for
// the stream-K kernel below).
template <int KV_DT, bool PAIR>
__global__ __launch_bounds__(kDecWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void
paged_decode_mfma16_2w_kernel(DecodeArgs a) {
  split_decode<KV_DT, PAIR>(a);
}

// ---------------------------------------------------------------------------
// Workgroup split (small batches): one workgroup per (sequence, KV head).
// Its nw waves take consecutive tile ranges of the sequence, run the split-K
// tile pipeline above, and merge their (acc, m, l) through LDS with the
// log-sum-exp rule; one pass writes the output.  No workspace, no second
// kernel: a batch of a few dozen sequences is bound by the latency of each
// wave's tile chain, and this shortens the chain by nw without the partial
// round trip through HBM and the merge launch.
// LDS (dynamic): acc [nw][group][head_dim] fp32, then m [nw][group], l [nw][group].
// ---------------------------------------------------------------------------
constexpr int kWgMaxWaves = 8;

// The LDS merge of the workgroup route: every wave writes its (acc, m, l)
// (lane (kg, c) holds O[head 4kg + r][dim 8c + mm] in acc[mm][r], m and l of
// head c), then the workgroup combines the nw partials of each (head, 8-dim
// chunk) with the log-sum-exp rule and writes the output row.  v_mul: the
// per-tensor V scale (1 otherwise).
template <bool PAIR>
MKV_DEV void wg_merge_store(const DecodeArgs& a, const WorkItem& it, const f32x4 (&acc)[8], float m_run,
                            float l_col, float v_mul) {
  extern __shared__ float wg_lds[];
  const int nw = blockDim.x >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  const int G = a.group;
  float* acc_l = wg_lds;
  float* m_l = wg_lds + nw * G * kHeadDim;
  float* l_l = m_l + nw * G;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * kg + r;
    if (h < G) {
      float* p = acc_l + (wv * G + h) * kHeadDim + 8 * c;
      *reinterpret_cast<f32x4*>(p) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      *reinterpret_cast<f32x4*>(p + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
    }
  }
  if (kg == 0 && c < G) {
    m_l[wv * G + c] = m_run;
    l_l[wv * G + c] = l_col;
  }
  __syncthreads();
  for (int u = threadIdx.x; u < G * 16; u += blockDim.x) {
    const int h = u >> 4, d0 = (u & 15) * 8;
    int col0;
    if (!out_cols<PAIR>(G, h, u & 15, col0)) continue;  // the other half of a paired head
    float M = kNegBig;
    for (int w = 0; w < nw; ++w) M = fmaxf(M, m_l[w * G + h]);
    float lsum = 0.0f, o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = 0.0f;
    for (int w = 0; w < nw; ++w) {
      const float e = __builtin_amdgcn_exp2f(m_l[w * G + h] - M);
      lsum += e * l_l[w * G + h];
      const float* p = acc_l + (w * G + h) * kHeadDim + d0;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(p);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o[j] += e * x0[j];
        o[4 + j] += e * x1[j];
      }
    }
    const float inv = lsum > 0.0f ? v_mul / lsum : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= inv;
    store_out8(a.out, a.q_dtype,
               (int64_t)it.b * a.out_stride + (int64_t)(it.kvh * G + h) * kQDim<PAIR> + col0, o);
  }
}

// Work item of wave wv of the workgroup route: the sequence's 32-token tiles
// cut into nw consecutive ranges.
MKV_DEV WorkItem wg_item(const DecodeArgs& a) {
  const int nw = blockDim.x >> 6;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  WorkItem it;
  it.b = (int)(blockIdx.x / (unsigned)a.num_kv_heads);
  it.kvh = (int)blockIdx.x - it.b * a.num_kv_heads;
  int64_t L = load_index(a.context_lens, it.b, a.ctx_i64);
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  const int tiles = (int)((L + 31) >> 5);
  const int per = (tiles + nw - 1) / nw;
  const int64_t tb = (int64_t)wv * per * 32, te = tb + (int64_t)per * 32;
  it.t_begin = (int)(tb < L ? tb : L);
  it.t_end = (int)(te < L ? te : L);
  it.split = wv;
  it.num_splits = nw;
  return it;
}

// Work of wave wv of the workgroup route: the sequence's 32-token tiles wv,
// wv + nw, wv + 2nw, ...  Dealt round robin, a wave's first tile does not
// depend on the context length, so its block-table entries and K/V loads go
// out in the same round trip as the length's own load: t_end starts at the
// table's capacity and is set when the length arrives.
MKV_DEV WorkItem wg_item_rr(const DecodeArgs& a) {
  WorkItem it;
  it.num_splits = blockDim.x >> 6;
  it.split = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  it.b = (int)(blockIdx.x / (unsigned)a.num_kv_heads);
  it.kvh = (int)blockIdx.x - it.b * a.num_kv_heads;
  it.t_begin = 32 * it.split;
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  it.t_end = (int)(cap < 0x7fffffff ? cap : 0x7fffffff);
  return it;
}

// Zero the V rows of a tile at or past t_end (token t0 + 16hf + 4kg + r in
// V word 4hf + r).  A tile loaded before the context length was known may
// hold stale pool bytes there, and a NaN among them would survive its zero
// weight in the PV product.  K rows need nothing: their scores are replaced
// by -inf.
template <int KV_DT>
MKV_DEV void zero_v_rows_past(Tile16<KV_DT>& T, int t0, int t_end) {
  const int kg = (threadIdx.x & 63) >> 4;
  using VT = typename Tile16<KV_DT>::VT;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool keep = t0 + 16 * (i >> 2) + 4 * kg + (i & 3) < t_end;
    T.v[i] = keep ? T.v[i] : VT{};
  }
}

// The workgroup route over 1-byte caches (FP8, per-token-head FP8 / INT8).
// Start-up in two round trips: a 16-bit q's loads, the context length, the
// first tile's block-table entries (scalar loads) and then that tile's K/V
// loads are issued before anything is waited for; the second tile's loads go
// out as soon as the length is known, and q is converted after them.
template <int KV_DT, bool PAIR, bool QS>
MKV_DEV void wg_decode_rr(const DecodeArgs& a) {
  WorkItem it = wg_item_rr(a);
  const int step = 32 * it.num_splits;
  const bool q16 = a.q_dtype != MKV_DTYPE_F32;
  QOps<KV_DT> qop;
  QStage qs;
  float score_mul = 0.0f;
  const float k_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.k_scale) : 1.0f;
  if (q16)
    load_q_stage<PAIR>(a, it.b, it.kvh, true, qs);
  else
    score_mul = load_q_operands<KV_DT, PAIR>(a, it.b, it.kvh, qop, k_mul);
  const int64_t L_raw = load_index(a.context_lens, it.b, a.ctx_i64);
  const ItemLoad Ld = item_load_setup<KV_DT>(a, it);
  // (two tiles in flight, as in the other routes: a third measured 1-2 us
  // slower on the engine's decode shapes)
  Tile16<KV_DT> ta, tb2;
  load_tile16<KV_DT, PAIR>(a, it, Ld, it.t_begin, item_phys(a, it.b, it.t_begin, it.t_end), ta);
  it.t_end = (int)(L_raw < 0 ? 0 : (L_raw < it.t_end ? L_raw : it.t_end));
  const bool hi = PAIR && (threadIdx.x & 15) >= (a.group >> 1);
  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;
  if (it.t_begin < it.t_end) {
    PhysPair ph = item_phys(a, it.b, it.t_begin + step, it.t_end);
    load_tile16<KV_DT, PAIR>(a, it, Ld, it.t_begin + step, ph, tb2);
    ph = item_phys(a, it.b, it.t_begin + 2 * step, it.t_end);
    if (q16) score_mul = staged_q_operands<KV_DT>(a, qs, qop, k_mul);
    qop.split = QS;
    zero_v_rows_past<KV_DT>(ta, it.t_begin, it.t_end);
    compute_tile16<KV_DT, PAIR>(ta, it.t_begin, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
    for (int t0 = it.t_begin + step; t0 < it.t_end;) {
      load_tile16<KV_DT, PAIR>(a, it, Ld, t0 + step, ph, ta);
      ph = item_phys(a, it.b, t0 + 2 * step, it.t_end);
      compute_tile16<KV_DT, PAIR>(tb2, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += step;
      if (t0 >= it.t_end) break;
      load_tile16<KV_DT, PAIR>(a, it, Ld, t0 + step, ph, tb2);
      ph = item_phys(a, it.b, t0 + 2 * step, it.t_end);
      compute_tile16<KV_DT, PAIR>(ta, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += step;
    }
  } else {
    // no tile in the context: let the speculative loads land before the
    // registers they write are reused
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  }
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  const float v_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.v_scale) : 1.0f;
  wg_merge_store<PAIR>(a, it, acc, m_run, l_col, v_mul);
}

// The workgroup route over 16-bit caches: consecutive tile ranges, started
// once the context length is known.  (Their tiles take twice the registers
// of the 1-byte formats', and the kernel sits at the two-waves-per-SIMD
// limit: the round-robin form below spills 8-14 registers here.)
template <int KV_DT, bool PAIR, bool QS>
MKV_DEV void wg_decode_contig(const DecodeArgs& a) {
  const WorkItem it = wg_item(a);

  QOps<KV_DT> qop;
  const float k_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.k_scale) : 1.0f;
  const float score_mul = load_q_operands<KV_DT, PAIR>(a, it.b, it.kvh, qop, k_mul);
  qop.split = QS;
  const bool hi = PAIR && (threadIdx.x & 15) >= (a.group >> 1);
  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;
  if (it.t_begin < it.t_end) {
    const ItemLoad Ld = item_load_setup<KV_DT>(a, it);
    Tile16<KV_DT> ta, tb2;
    load_tile16<KV_DT, PAIR>(a, it, Ld, it.t_begin, item_phys(a, it.b, it.t_begin, it.t_end), ta);
    PhysPair ph = item_phys(a, it.b, it.t_begin + 32, it.t_end);
    for (int t0 = it.t_begin;;) {
      load_tile16<KV_DT, PAIR>(a, it, Ld, t0 + 32, ph, tb2);
      ph = item_phys(a, it.b, t0 + 64, it.t_end);
      compute_tile16<KV_DT, PAIR>(ta, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += 32;
      if (t0 >= it.t_end) break;
      load_tile16<KV_DT, PAIR>(a, it, Ld, t0 + 32, ph, ta);
      ph = item_phys(a, it.b, t0 + 64, it.t_end);
      compute_tile16<KV_DT, PAIR>(tb2, t0, it.t_end, qop, score_mul, acc, m_run, l_run, hi);
      t0 += 32;
      if (t0 >= it.t_end) break;
    }
  }
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  const float v_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.v_scale) : 1.0f;
  wg_merge_store<PAIR>(a, it, acc, m_run, l_col, v_mul);
}

// QS: the q split of the bf16 MFMA formats (an fp32 / fp16 q over a bf16 or
// per-token-head cache) as a compile-time choice, so that the common case
// (a bf16 q) holds no residual terms.
template <int KV_DT, bool PAIR, bool QS>
MKV_DEV void wg_decode(const DecodeArgs& a) {
  if constexpr (DTypeInfo<KV_DT>::kBytes == 2)
    wg_decode_contig<KV_DT, PAIR, QS>(a);
  else
    wg_decode_rr<KV_DT, PAIR, QS>(a);
}

template <int KV_DT, bool PAIR>
__global__ __launch_bounds__(kWgMaxWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void
paged_decode_wg_kernel(DecodeArgs a) {
  wg_decode<KV_DT, PAIR, false>(a);
}

// The split-q variant of the bf16 MFMA formats holds 16 more registers of q
// than two waves per SIMD leave room for: it runs at one wave per SIMD with
// at most kWgSplitWaves waves per workgroup (a workgroup still fits one CU).
constexpr int kWgSplitWaves = 4;
template <int KV_DT, bool PAIR>
__global__ __launch_bounds__(kWgSplitWaves* kWave) void paged_decode_wg_qsplit_kernel(DecodeArgs a) {
  wg_decode<KV_DT, PAIR, true>(a);
}

// ---------------------------------------------------------------------------
// A decode step's producer and attention in one launch (per-tensor FP8
// caches, head_dim 128).  Per layer, the reference's decode step runs the
// q/k norm, rotary embedding and append of every sequence's new token
// (qwen3.py:73-118, attention.py:1654-1691) and then the decode attention
// over the cache that now holds it (attention.py:1213-1268).  Here the
// workgroup of (sequence b, KV head kvh) of the workgroup route does both:
// its waves share out the token's q heads of the group and its K and V
// heads kvh (one head per wave pass, 64 lanes wide, with the producer
// kernel's operations in the producer kernel's order), put q and the new
// K / V cache rows in LDS, and append the rows.  Per-tensor FP8: the first
// tile's loads go out before the producer's math, the second tile's after
// the barrier, either before the append lands, and the wave whose tile
// holds the token's position takes that row from LDS instead of from the
// cache.  Per-token-head caches: the first tile goes out early and the
// wave that holds the token's position loads it again once the append has
// landed.  16-bit caches: every tile is loaded after the append has
// landed.  The result is the producer kernel followed by the workgroup
// route, bit for bit.
// LDS (dynamic): the workgroup merge area of wg_merge_store, then q of the
// group's heads (fp32 [G][128]) and the new token's K row and V row (128
// elements each in the cache dtype).
// ---------------------------------------------------------------------------
constexpr int kFusedMaxGroup = 8;  // query heads per KV head

struct ProduceDecodeArgs {
  DecodeArgs d;    // the attention (d.q is not read: q comes from the producer step)
  ProducerArgs p;  // the producer step of the batch's one token per sequence
};

// Replace row p (0..31, wave-uniform) of an FP8 tile, as loaded (before
// k_exchange), with the new token's K / V row at kv in LDS (the cache row's
// bytes of this KV head: K, then V).  Load A of sub-tile m holds row c & 7,
// bytes 32kg + (c < 8 ? 0 : 16); load B row (c & 7) + 8, bytes
// 32kg + (c < 8 ? 16 : 0) (fp8_k_lanes); V word i: row 16 (i >> 2) + 4kg +
// (i & 3), bytes 8c .. 8c+7.  (Selects, not branches: a tile changed on two
// paths lands in scratch memory.)
template <int KV_DT>
MKV_DEV void patch_tile_row(Tile16<KV_DT>& T, int p, const unsigned char* kv) {
  static_assert(DTypeInfo<KV_DT>::kBytes == 1, "1-byte caches");
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  const bool top = c < 8;
  const u32x4 na = *reinterpret_cast<const u32x4*>(kv + 32 * kg + (top ? 0 : 16));
  const u32x4 nb = *reinterpret_cast<const u32x4*>(kv + 32 * kg + (top ? 16 : 0));
  const u32x2 nv = *reinterpret_cast<const u32x2*>(kv + 128 + 8 * c);
  const int r = p & 15;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const bool sub = (p >> 4) == m;
    T.k[m][0] = sub && r < 8 && (c & 7) == r ? na : T.k[m][0];
    T.k[m][1] = sub && r >= 8 && (c & 7) == r - 8 ? nb : T.k[m][1];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) T.v[i] = 16 * (i >> 2) + 4 * kg + (i & 3) == p ? nv : T.v[i];
}

// Raw word holding element i of a dtype-dt row at p (the element's own
// dword for fp32, the aligned dword of its pair for 16-bit types), and the
// element in fp32 (exact, as load8_f32 gives it).
MKV_DEV uint32_t elem_word(const char* p, int i, int dt) {
  return *reinterpret_cast<const uint32_t*>(p + (dt == MKV_DTYPE_F32 ? 4 * i : ((2 * i) & ~3)));
}
MKV_DEV float word_elem(uint32_t w, int i, int dt) {
  const uint32_t h = (i & 1) ? w >> 16 : w & 0xffffu;
  const float x16 = dt == MKV_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
  return dt == MKV_DTYPE_F32 ? __uint_as_float(w) : x16;
}

// The FP8 code of one element at a per-tensor scale (quantize4_fp8's byte).
MKV_DEV uint32_t fp8_code(float x, const Fp8Quant& q) {
  const float v[4] = {x, 0.0f, 0.0f, 0.0f};
  return quantize4_fp8(v, q) & 0xffu;
}

// KV_DT: MKV_DTYPE_FP8E4M3 (per-tensor scales), a per-token-head FP8 /
// INT8 format (one scale per slot and KV head, from the head's amax, as
// store_kv writes it) or a 16-bit cache (copy append, cast to the cache
// dtype).  1-byte caches take the workgroup route's round-robin tiles
// (wg_decode_rr; per-tensor FP8 with its speculative first tile), 16-bit
// caches its consecutive ranges (wg_decode_contig).
template <int IN_DT, int KV_DT>
MKV_DEV void wg_produce_decode(const ProduceDecodeArgs& f) {
  constexpr bool kFp8 = KV_DT == MKV_DTYPE_FP8E4M3;
  constexpr bool kTok = kPerTokenScale<KV_DT>;
  constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  constexpr int kIb = DTypeInfo<IN_DT>::kBytes;
  extern __shared__ float wg_lds[];
  const DecodeArgs& a = f.d;
  const ProducerArgs& pa = f.p;
  WorkItem it = wg_item_rr(a);
  const int nw = it.num_splits, wv = it.split;
  const int lane = threadIdx.x & 63;
  const int G = a.group;

  // The producer step of token b for KV head kvh, one head per wave pass:
  // head slot hs < G is q head kvh * G + hs, hs == G the k head, hs == G + 1
  // the v head; wave wv takes slots wv, wv + nw, ...; lane l holds elements
  // l and 64 + l of the slot's head (a rotary pair).  The loads of a wave's
  // first two slots depend on nothing: they go out before anything else.
  const char* row = pa.qkv + it.b * pa.qkv_stride * kIb;
  auto head_row = [&](int hs) -> const char* {
    const int head = hs < G ? it.kvh * G + hs
                            : (hs == G ? a.num_heads + it.kvh : a.num_heads + a.num_kv_heads + it.kvh);
    return row + (int64_t)head * kHeadDim * kIb;
  };
  // (no weight: the row stands in as a readable address; unused)
  auto weight = [&](int hs) -> const char* {
    const void* w = hs < G ? pa.q_w : pa.k_w;
    return w ? reinterpret_cast<const char*>(w) : row;
  };
  struct SlotIn {
    uint32_t x1, x2, w1, w2;
  };
  auto slot_loads = [&](int hs) {
    const int h = hs < G + 2 ? hs : G + 1;
    const char* hr = head_row(h);
    const char* w = weight(h);
    return SlotIn{elem_word(hr, lane, IN_DT), elem_word(hr, 64 + lane, IN_DT), elem_word(w, lane, pa.w_dtype),
                  elem_word(w, 64 + lane, pa.w_dtype)};
  };
  const SlotIn in0 = slot_loads(wv), in1 = slot_loads(wv + nw);

  // Scalars: the context length, the token's position and slot, the
  // per-tensor scales (the stored values, or the calibration of this call's
  // rows while the 1.0 sentinel is there: every wave computes the same value,
  // as the producer kernel's waves do).
  const int64_t L_raw = load_index(a.context_lens, it.b, a.ctx_i64);
  const int64_t pos = pa.positions[it.b];
  const int64_t slot = pa.slot_mapping[it.b];
  float ks = 1.0f, vs = 1.0f;
  if constexpr (kFp8) {
    ks = load_uniform_f32(pa.k_scale);
    vs = load_uniform_f32(pa.v_scale);
    if (pa.calibrate && (ks == 1.0f || vs == 1.0f)) {
      const int m = lane & 7, wb = dtype_bytes(pa.w_dtype);
      float wkl[8] = {}, wkh[8] = {};
      if (pa.k_w) {
        load8_f32(reinterpret_cast<const char*>(pa.k_w) + (8 * m) * wb, pa.w_dtype, wkl);
        load8_f32(reinterpret_cast<const char*>(pa.k_w) + (64 + 8 * m) * wb, pa.w_dtype, wkh);
      }
      if (ks == 1.0f) ks = producer_calibrate(pa, true, pa.k_scale, IN_DT, wkl, wkh);
      if (vs == 1.0f) vs = producer_calibrate(pa, false, pa.v_scale, IN_DT, wkl, wkh);
      // vmcnt(0) before the paths join: with this branch's loads pending
      // there, the compiler's wait at the join also held every call's tile
      // loads back until the producer's loads had returned
      __builtin_amdgcn_s_waitcnt(0x0f70);
    }
  }
  const bool append = slot >= 0 && slot < pa.num_slots;
  // The cos / sin pair of the position (rotary_row's values), issued before
  // any tile's loads: the load counter returns loads in issue order, and the
  // producer's math waits only for its own inputs.
  const bool pos_ok = pos >= 0 && pos < pa.max_position;
  const char* csr = reinterpret_cast<const char*>(pa.cos_sin) +
                    (pos_ok ? pos : 0) * kHeadDim * dtype_bytes(pa.cs_dtype);
  const uint32_t cw = elem_word(csr, lane, pa.cs_dtype), sw = elem_word(csr, 64 + lane, pa.cs_dtype);

  // The first tile: per-tensor FP8 loads it speculatively (as in
  // wg_decode_rr); per-token-head caches take the same round-robin tiles,
  // 16-bit caches consecutive ranges, known once the context length is
  // (wg_item's split), both loaded after the append.
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  const int64_t L = L_raw < 0 ? 0 : (L_raw > cap ? cap : L_raw);
  int step = 32 * nw;
  if constexpr (kTok) it.t_end = (int)(L < it.t_end ? L : it.t_end);
  if constexpr (kEb == 2) {
    const int tiles = (int)((L + 31) >> 5);
    const int per = (tiles + nw - 1) / nw;
    const int64_t tb = (int64_t)wv * per * 32, te = tb + (int64_t)per * 32;
    it.t_begin = (int)(tb < L ? tb : L);
    it.t_end = (int)(te < L ? te : L);
    step = 32;
  }
  const ItemLoad Ld = item_load_setup<KV_DT>(a, it);
  Tile16<KV_DT> ta, tb2;
  PhysPair ph = item_phys(a, it.b, it.t_begin, it.t_end);
  if constexpr (kFp8 || kTok) load_tile16<KV_DT, false>(a, it, Ld, it.t_begin, ph, ta);
  const PhysPair ph_first = ph;

  // Per-tensor FP8: the context length is known; the second tile's
  // block-table entries are looked up here and its loads go out after the
  // barrier.  A wave issues in order, and while the grid's first tiles are
  // in flight a load's issue stalls: 12 more loads ahead of the producer's
  // math held back the math and the barrier that every wave of the
  // workgroup waits at (the step measured 20.1 us with them there, 19.2-19.3
  // us with them after the barrier, at 60 rows of 300-800 tokens).  The new
  // token's row is patched into the tile that holds position L - 1 when
  // this call appends it there (slot = that position's cache row): that
  // tile's loads may have left before the append landed.  Per-token-head
  // caches issue the first tile early too and, instead of a patch (it would
  // need the row's scales as well), the wave whose first tile holds
  // position L - 1 loads that tile again after the barrier, once the waves
  // that appended have waited for their stores (the others keep their
  // loads in flight: 24.1-24.7 -> 23.4 us at 60 rows of 300-800 tokens).
  // 16-bit caches load every tile after the append has landed (the patch's
  // registers beside two 16-bit tiles would spill).
  bool patch = false;
  const int pl = (int)L - 1;
  if constexpr (kFp8) {
    it.t_end = (int)(L < it.t_end ? L : it.t_end);
    const int64_t phys_pl = pl >= 0 ? a.idx.physical_block(it.b, pl >> a.idx.bs_log2) : -1;
    patch = append && phys_pl >= 0 && (phys_pl << a.idx.bs_log2) + (pl & ((1 << a.idx.bs_log2) - 1)) == slot;
    ph = item_phys(a, it.b, it.t_begin + step, it.t_end);
  }

  // The producer's math (produce_qk / load_v and store_kv's bytes, the same
  // operations in the same order): q into the workgroup's q area (fp32
  // [G][128]), the new token's K and V cache rows of head kvh into its row
  // area (2 x 128 x kEb bytes), and the wave of the k / v slot appends them.
  float* qsh = wg_lds + nw * G * (kHeadDim + 2);
  uint32_t* kvsh = reinterpret_cast<uint32_t*>(qsh + G * kHeadDim);  // [K row | V row]
  constexpr int kRowWords = kHeadDim * kEb / 4;
  const float c = pos_ok ? word_elem(cw, lane, pa.cs_dtype) : __builtin_nanf("");
  const float sn = pos_ok ? word_elem(sw, lane, pa.cs_dtype) : __builtin_nanf("");
  auto produce = [&](int hs, const SlotIn& in) {
    // (products that feed a sum through mul_rn, as in norm_rope)
    float o1 = word_elem(in.x1, lane, IN_DT), o2 = word_elem(in.x2, lane, IN_DT);
    if (hs <= G) {
      float x1 = o1, x2 = o2;
      if (hs < G ? pa.q_w != nullptr : pa.k_w != nullptr) {
        // norm: the sum of squares in produce_qk's order (pair 8m + j of lane
        // m, j = 0..7 in turn, then a butterfly over m)
        const float t = __fadd_rn(mul_rn(x1, x1), mul_rn(x2, x2));
        const int base = lane & ~7;
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __fadd_rn(ss, __shfl(t, base + j));
        ss = ss + __shfl_xor(ss, 8);
        ss = ss + __shfl_xor(ss, 16);
        ss = ss + __shfl_xor(ss, 32);
        const float var = __fadd_rn(ss / (float)pa.head_dim, pa.eps);  // (a division, as in norm_rope)
        const float r = sqrtf(var);
        x1 = round_to_dtype(__fmul_rn(x1 / r, word_elem(in.w1, lane, pa.w_dtype)), IN_DT);
        x2 = round_to_dtype(__fmul_rn(x2 / r, word_elem(in.w2, lane, pa.w_dtype)), IN_DT);
      }
      o1 = round_to_dtype(__fsub_rn(mul_rn(x1, c), mul_rn(x2, sn)), pa.out_dtype);
      o2 = round_to_dtype(__fadd_rn(mul_rn(x1, sn), mul_rn(x2, c)), pa.out_dtype);
    }
    if (hs < G) {
      qsh[hs * kHeadDim + lane] = o1;
      qsh[hs * kHeadDim + 64 + lane] = o2;
    } else if (hs < G + 2) {
      // the cache bytes of elements l and 64 + l, gathered to words (4 FP8
      // codes or 2 16-bit values)
      uint32_t w1, w2;
      bool lead;
      if constexpr (kEb == 1) {
        // per-tensor: the tensor's scale; per token and head: store_kv's
        // scale of the head's amax (exact whatever the order), stored by one
        // lane, and its codes
        uint32_t b1, b2;
        if constexpr (kTok) {
          const float am = wave_max(fmaxf(fmaxf(0.0f, fabsf(o1)), fabsf(o2)));
          const float hsc = KV_DT == kKvI8PerToken ? i8_head_scale(am) : fp8_head_scale(am);
          if constexpr (KV_DT == kKvI8PerToken) {
            const float inv = 1.0f / hsc;
            b1 = quantize_i8(o1, inv) & 0xffu;
            b2 = quantize_i8(o2, inv) & 0xffu;
          } else {
            const Fp8Quant qz = fp8_quant(hsc);
            b1 = fp8_code(o1, qz);
            b2 = fp8_code(o2, qz);
          }
          if (append && lane == 0) (hs == G ? pa.k_scale : pa.v_scale)[slot * pa.num_kv_heads + it.kvh] = hsc;
        } else {
          const Fp8Quant qz = fp8_quant(hs == G ? ks : vs);
          b1 = fp8_code(o1, qz);
          b2 = fp8_code(o2, qz);
        }
        w1 = b1 | (uint32_t)__shfl(b1, lane + 1) << 8 | (uint32_t)__shfl(b1, lane + 2) << 16 |
             (uint32_t)__shfl(b1, lane + 3) << 24;
        w2 = b2 | (uint32_t)__shfl(b2, lane + 1) << 8 | (uint32_t)__shfl(b2, lane + 2) << 16 |
             (uint32_t)__shfl(b2, lane + 3) << 24;
        lead = (lane & 3) == 0;
      } else {
        const bool bf = KV_DT == MKV_DTYPE_BF16;
        const uint32_t h1 = bf ? f32_to_bf16_bits(o1) : f32_to_f16_bits(o1);
        const uint32_t h2 = bf ? f32_to_bf16_bits(o2) : f32_to_f16_bits(o2);
        w1 = h1 | (uint32_t)__shfl(h1, lane + 1) << 16;
        w2 = h2 | (uint32_t)__shfl(h2, lane + 1) << 16;
        lead = (lane & 1) == 0;
      }
      if (lead) {
        const int wi = lane * kEb / 4;  // word of element l in the row
        uint32_t* dst = kvsh + (hs == G ? 0 : kRowWords);
        dst[wi] = w1;
        dst[kRowWords / 2 + wi] = w2;
        if (append) {
          char* base = (hs == G ? pa.k_cache : pa.v_cache) + (slot * a.idx.row_elems + (int64_t)it.kvh * kHeadDim) * kEb;
          *reinterpret_cast<uint32_t*>(base + lane * kEb) = w1;
          *reinterpret_cast<uint32_t*>(base + (64 + lane) * kEb) = w2;
        }
      }
    }
  };
  produce(wv, in0);
  produce(wv + nw, in1);
  for (int hs = wv + 2 * nw; hs < G + 2; hs += nw) produce(hs, slot_loads(hs));
  // vmcnt(0): the append has landed.  Per-token-head: only in the waves that
  // appended (their first tiles' loads stay in flight in the others).
  const bool appended = append && ((G >= wv && (G - wv) % nw == 0) || (G + 1 - wv) % nw == 0);
  if constexpr (kTok) {
    if (appended) __builtin_amdgcn_s_waitcnt(0x0f70);
  } else if constexpr (!kFp8) {
    __builtin_amdgcn_s_waitcnt(0x0f70);
  }
  __syncthreads();  // q and the new K / V row are in LDS (16-bit: and in the cache)
  const unsigned char* kv_new = reinterpret_cast<const unsigned char*>(kvsh);
  if constexpr (kTok) {
    // The first tile went out before the append: the wave whose first tile
    // holds position L - 1 loads it (codes and scales) again
    if (pl >= it.t_begin && pl < it.t_begin + 32) load_tile16<KV_DT, false>(a, it, Ld, it.t_begin, ph_first, ta);
    ph = item_phys(a, it.b, it.t_begin + step, it.t_end);
    load_tile16<KV_DT, false>(a, it, Ld, it.t_begin + step, ph, tb2);
    ph = item_phys(a, it.b, it.t_begin + 2 * step, it.t_end);
  } else if constexpr (!kFp8) {
    load_tile16<KV_DT, false>(a, it, Ld, it.t_begin, ph, ta);
    ph = item_phys(a, it.b, it.t_begin + step, it.t_end);
    load_tile16<KV_DT, false>(a, it, Ld, it.t_begin + step, ph, tb2);
    ph = item_phys(a, it.b, it.t_begin + 2 * step, it.t_end);
  }

  auto fix = [&](Tile16<KV_DT>& T, int t0) {
    if constexpr (kFp8)
      if (patch && pl >= t0 && pl < t0 + 32) patch_tile_row<KV_DT>(T, pl - t0, kv_new);
  };
  QOps<KV_DT> qop;
  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;
  if (it.t_begin < it.t_end) {
    if constexpr (kFp8) {  // the second tile (empty past the range)
      load_tile16<KV_DT, false>(a, it, Ld, it.t_begin + step, ph, tb2);
      ph = item_phys(a, it.b, it.t_begin + 2 * step, it.t_end);
    }
    // q of head c, dims 32kg .. 32kg+31 (zeros for padding heads)
    const int cq = lane & 15, kg = lane >> 4;
    float qf[32];
    const float* q = qsh + (cq < G ? cq : 0) * kHeadDim + 32 * kg;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(q + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) qf[4 * i + j] = cq < G ? x[j] : 0.0f;
    }
    const float score_mul = q_operands<KV_DT>(a, qf, qop, ks);
    qop.split = false;
    if constexpr (kFp8) zero_v_rows_past<KV_DT>(ta, it.t_begin, it.t_end);
    fix(ta, it.t_begin);
    compute_tile16<KV_DT, false>(ta, it.t_begin, it.t_end, qop, score_mul, acc, m_run, l_run, false);
    for (int t0 = it.t_begin + step; t0 < it.t_end;) {
      load_tile16<KV_DT, false>(a, it, Ld, t0 + step, ph, ta);
      ph = item_phys(a, it.b, t0 + 2 * step, it.t_end);
      fix(tb2, t0);
      compute_tile16<KV_DT, false>(tb2, t0, it.t_end, qop, score_mul, acc, m_run, l_run, false);
      t0 += step;
      if (t0 >= it.t_end) break;
      load_tile16<KV_DT, false>(a, it, Ld, t0 + step, ph, tb2);
      ph = item_phys(a, it.b, t0 + 2 * step, it.t_end);
      fix(ta, t0);
      compute_tile16<KV_DT, false>(ta, t0, it.t_end, qop, score_mul, acc, m_run, l_run, false);
      t0 += step;
    }
  } else {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the loads in flight land first
  }
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  wg_merge_store<false>(a, it, acc, m_run, l_col, vs);
}

template <int IN_DT, int KV_DT>
__global__ __launch_bounds__(kWgMaxWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void
paged_decode_wg_produce_kernel(ProduceDecodeArgs f) {
  wg_produce_decode<IN_DT, KV_DT>(f);
}

// fp32 caches on the workgroup route: 16-token tiles on v_mfma_f32_16x16x4_f32
// (the split-K fp32 kernel's arithmetic), loaded through per-tile buffer
// descriptors one tile ahead of the math.
struct TileF32 {
  u32x4 k[8];     // K row of token t0 + c, dims 32kg .. 32kg+31
  u32x4 v[4][2];  // V rows of tokens t0 + 4kg + r, dims 8c .. 8c+7
  bool ok;        // block present
};

// The loads of the 16-token tile at t0 in block phys (item_phys1).
MKV_DEV void load_tile_f32(const DecodeArgs& a, const WorkItem& it, const ItemLoad& L, int t0, int64_t phys,
                           TileF32& T) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  const int bs_mask = (1 << a.idx.bs_log2) - 1;
  const int64_t off = L.head_bytes + (int64_t)(t0 & bs_mask) * L.row_bytes;
  const __amdgpu_buffer_rsrc_t rk = rows_rsrc(a.k_cache, phys, L.blk_bytes, off);
  const __amdgpu_buffer_rsrc_t rv = rows_rsrc(a.v_cache, phys, L.blk_bytes, off);
  T.ok = phys >= 0;
  const uint32_t ko = (t0 + c < it.t_end) ? (uint32_t)L.k_voff : kOob;
#pragma unroll
  for (int i = 0; i < 8; ++i) T.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 16 * i, 0, kAuxNt);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t vo = (t0 + 4 * kg + r < it.t_end) ? (uint32_t)(L.v_voff + r * L.row_bytes) : kOob;
    T.v[r][0] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, kAuxNt);
    T.v[r][1] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo + 16, 0, kAuxNt);
  }
}

MKV_DEV void compute_tile_f32(const TileF32& T, int t0, int t_end, const float (&qf)[32], float score_mul,
                              f32x4 (&acc)[8], float& m_run, float& l_run) {
  const int kg = (threadIdx.x & 63) >> 4;
  f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 32; ++st)
    s = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(T.k[st >> 2][st & 3]), qf[st], s, 0, 0, 0);
  float mx = kNegBig;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool ok = t0 + 4 * kg + r < t_end && T.ok;
    s[r] = ok ? s[r] * score_mul : -__builtin_huge_valf();
    mx = fmaxf(mx, s[r]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = fmaxf(m_run, mx);
  const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
  m_run = m_new;
  float p[4], psum = 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
    psum += p[r];
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
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int mm = 0; mm < 8; ++mm)
      acc[mm] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[r], __uint_as_float(T.v[r][mm >> 2][mm & 3]), acc[mm],
                                                      0, 0, 0);
  }
}

// The fp32 tile pipeline of one wave over its range [t_begin, t_end): the
// loads of tile i+1 in flight while tile i is computed, the block-table entry
// of tile i+2 (a scalar load) while tile i+1's loads go out.
MKV_DEV void f32_range(const DecodeArgs& a, const WorkItem& it, const float (&qf)[32], float score_mul,
                       f32x4 (&acc)[8], float& m_run, float& l_run) {
  if (it.t_begin >= it.t_end) return;
  const ItemLoad Ld = item_load_setup<MKV_DTYPE_F32>(a, it);
  TileF32 ta, tb;
  load_tile_f32(a, it, Ld, it.t_begin, item_phys1(a, it.b, it.t_begin, it.t_end), ta);
  int64_t ph = item_phys1(a, it.b, it.t_begin + 16, it.t_end);
  for (int t0 = it.t_begin;;) {
    load_tile_f32(a, it, Ld, t0 + 16, ph, tb);
    ph = item_phys1(a, it.b, t0 + 32, it.t_end);
    compute_tile_f32(ta, t0, it.t_end, qf, score_mul, acc, m_run, l_run);
    t0 += 16;
    if (t0 >= it.t_end) break;
    load_tile_f32(a, it, Ld, t0 + 16, ph, ta);
    ph = item_phys1(a, it.b, t0 + 32, it.t_end);
    compute_tile_f32(tb, t0, it.t_end, qf, score_mul, acc, m_run, l_run);
    t0 += 16;
    if (t0 >= it.t_end) break;
  }
}

// q of item (b, kvh) as fp32 for the fp32 kernels (same lane slice as the
// 16-bit kernels).
template <bool PAIR>
MKV_DEV void load_q_f32(const DecodeArgs& a, int b, int kvh, float (&qf)[32]) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  int d0;
  if (q_slice<PAIR>(a.group, c, kg, d0)) {
    const int64_t qoff = (int64_t)b * a.q_stride + (int64_t)(kvh * a.group + c) * kQDim<PAIR> + d0;
    load_q32(a.q, a.q_dtype, qoff, qf);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) qf[i] = 0.0f;
  }
}

template <bool PAIR>
__global__ __launch_bounds__(kWgMaxWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void
paged_decode_wg_f32_kernel(DecodeArgs a) {
  const WorkItem it = wg_item(a);
  float qf[32];
  load_q_f32<PAIR>(a, it.b, it.kvh, qf);
  const float score_mul = a.sm_scale * kLog2e;
  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;
  f32_range(a, it, qf, score_mul, acc, m_run, l_run);
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  wg_merge_store<PAIR>(a, it, acc, m_run, l_col, 1.0f);
}

// ---------------------------------------------------------------------------
// Stream-K decode (16-bit MFMA path, the default).
//
// The work is one global stream of columns: sequence by sequence, the
// ceil(L/32) 32-token tiles of every sequence, each column standing for that
// tile of all Hkv KV heads.  The persistent grid's W waves form W / Hkv
// groups of Hkv consecutive waves; the groups split the column stream into
// equal contiguous ranges, and wave k of a group computes KV head k of every
// column in its group's range.  So every wave streams the same number of
// bytes whatever the context-length skew, its load pipeline runs across item
// boundaries (the next tile's block-table entry and K/V are always in
// flight), and the Hkv heads' 128-byte slices of each 1 KB token row are read
// by the Hkv waves of one group at about the same time (walking one head over
// a long token range while the other heads of the same rows come much later
// measured 4% slower on a pure read of the pool layout).  An item (sequence,
// KV head) cut by a range boundary writes (acc, m, l) partials to slot
// (wave, 0) if it began at or before the range, else (wave, 1); the merge
// kernel combines them.  Sequences with no visible token are written as
// zeros by the merge kernel.
// ---------------------------------------------------------------------------
constexpr int kTileTok = 32;
constexpr int kStreamMaxBatch = 8192;
constexpr size_t kStreamMaxLds = (2 * kStreamMaxBatch + 1) * sizeof(int);
constexpr int kStreamSmallBatch = 2047;
// Finishes a wave may hold in LDS (batches up to kStreamDeferMaxBatch): each
// takes 64 lanes x 64 bytes plus 16 bytes per wave.  Holding the finishes
// before a range's last tile and storing them after it took the batch-256
// FP8 step from 6188 to 6304-6310 GB/s (one held: 6291).
constexpr int kStreamDefer = 3;
constexpr int kStreamDeferMaxBatch = 1024;
constexpr size_t stream_lds_bytes(int batch, int defer) {
  return ((size_t)(2 * batch + 1) * sizeof(int) + 15) / 16 * 16 +
         (size_t)defer * kDecWaves * (kWave * 64 + 16);
}
constexpr size_t kStreamSmallLds =
    stream_lds_bytes(kStreamSmallBatch, 0) > stream_lds_bytes(kStreamDeferMaxBatch, kStreamDefer)
        ? stream_lds_bytes(kStreamSmallBatch, 0)
        : stream_lds_bytes(kStreamDeferMaxBatch, kStreamDefer);
static_assert(kStreamSmallLds <= 65536, "stream-K dynamic LDS");

struct Cursor {
  int b, kvh, t;  // item (sequence, KV head) and tile index inside the item
  int n, L;       // tiles of the item, visible tokens of the sequence
};

MKV_DEV int lds_uniform(const int* p, int i) { return __builtin_amdgcn_readfirstlane(p[i]); }

// The next column of the same KV head.
MKV_DEV void cursor_next(Cursor& c, const int* pre, const int* lens, int B) {
  if (++c.t < c.n) return;
  c.t = 0;
  do {
    ++c.b;
  } while (c.b < B && lds_uniform(pre, c.b + 1) == lds_uniform(pre, c.b));
  if (c.b < B) {
    c.n = lds_uniform(pre, c.b + 1) - lds_uniform(pre, c.b);
    c.L = lds_uniform(lens, c.b);
  } else {  // past the stream: an empty item whose loads read nothing
    c.b = B - 1;
    c.n = 1;
    c.L = 0;
  }
}

// Block-table entries of the two 16-token halves of tile c (scalar loads).
MKV_DEV PhysPair tile_phys(const DecodeArgs& a, const Cursor& c) {
  PhysPair ph;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tok = c.t * kTileTok + 16 * h;
    ph.p[h] = tok < c.L ? a.idx.physical_block(c.b, tok >> a.idx.bs_log2) : -1;
  }
  return ph;
}

// Issue the K/V loads of tile c (same lane mapping as load_tile16).
template <int KV_DT, bool PAIR>
MKV_DEV void load_tile_sk(const DecodeArgs& a, const Cursor& c, const PhysPair& ph, int row_bytes,
                          int64_t blk_bytes, int k_voff, int v_voff, Tile16<KV_DT>& T) {
  constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  const int lane = threadIdx.x & 63;
  const int cc = lane & 15, kg = lane >> 4;
  const int bs_mask = (1 << a.idx.bs_log2) - 1;
  const int t0 = c.t * kTileTok;
  const int64_t head_bytes = (int64_t)c.kvh * kHeadDim * kEb;
  __amdgpu_buffer_rsrc_t rk[2], rv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t off = head_bytes + (int64_t)((t0 + 16 * h) & bs_mask) * row_bytes;
    rk[h] = rows_rsrc(a.k_cache, ph.p[h], blk_bytes, off);
    rv[h] = rows_rsrc(a.v_cache, ph.p[h], blk_bytes, off);
    T.ok[h] = ph.p[h] >= 0;
  }
  load_tile_rows<KV_DT>(rk, rv, t0, c.L, k_voff, v_voff, row_bytes, T);
  load_tile_scales<KV_DT, PAIR>(a, ph.p[0], ph.p[1], t0, c.kvh, T);
}

// Write the finished item of cursor c: the normalised output if the whole item
// ran in this wave, else a partial in slot (wave, k).
template <bool PAIR>
MKV_DEV void finish_sk(const DecodeArgs& a, const Cursor& c, bool whole, int w, int k,
                       f32x4 (&acc)[8], float m_col, float l_col, float v_mul) {
  const int lane = threadIdx.x & 63;
  const int cc = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * kg + r;
    const float lh = __shfl(l_col, h);
    const float mh = __shfl(m_col, h);
    if (h >= a.group) continue;
    if (whole) {
      const float inv = lh > 0.0f ? v_mul / lh : 0.0f;
      float x[8];
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) x[mm] = acc[mm][r] * inv;
      const int hq = c.kvh * a.group + h;
      int col0;
      if (out_cols<PAIR>(a.group, h, cc, col0))
        store_out8(a.out, a.q_dtype, (int64_t)c.b * a.out_stride + (int64_t)hq * kQDim<PAIR> + col0, x);
    } else {
      const int64_t slot = ((int64_t)w * 2 + k) * a.group + h;
      float* p = a.ws_acc + slot * kHeadDim + 8 * cc;
      u32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = __float_as_uint(acc[j][r]);
        hi[j] = __float_as_uint(acc[4 + j][r]);
      }
      st16(p, lo);
      st16(p + 4, hi);
      if (cc == 0) {
        a.ws_ml[slot * 2] = mh;
        a.ws_ml[slot * 2 + 1] = lh;
      }
    }
  }
}

// Finish of an item for groups of at most 4 query heads (8 with head
// pairing, whose heads own 64 dims each), issued as exactly three buffer
// stores on every pipeline step (an unused store gets an empty range and
// writes nothing), for the same reason as load_q_stage's need flag.  Heads
// live in lane group 0 (head r in acc[.][r]; with pairing head j in lane
// group j / 4, its own dims in lanes c < 8 or c >= 8); four shuffles per
// output register spread them so that every lane holds 8 dims of one head
// (lane group h: head h, or with pairing lane 8j + d: head j, its own dims
// 8d ..), and one 16-byte store per lane covers all heads.  Store A/B: the
// output (bf16/fp16: A only; fp32: A and B) or the fp32 partial accumulator;
// store C: the partial's (m, l).
struct FinishStores {
  __amdgpu_buffer_rsrc_t ra, rc;
  uint32_t oa, ob, oc;
  u32x4 da, db;
  u32x2 dc;
};

MKV_DEV void finish_none(FinishStores& f) {
  f.ra = __builtin_amdgcn_make_buffer_rsrc(nullptr, (short)0, 0, kRsrcFlags);
  f.rc = f.ra;
  f.oa = f.ob = f.oc = kOob;
}

// Store descriptors of an item's finish: its output row (whole) or its
// partial slot k of wave w (acc, then (m, l)).  All inputs wave-uniform.
template <bool PAIR>
MKV_DEV void finish_rsrc(const DecodeArgs& a, bool whole, int b, int kvh, int w, int k, FinishStores& f) {
  if (whole) {
    const int ob = a.q_dtype == MKV_DTYPE_F32 ? 4 : 2;
    const char* base = reinterpret_cast<const char*>(a.out) +
                       ((int64_t)b * a.out_stride + (int64_t)kvh * a.group * kQDim<PAIR>) * ob;
    f.ra = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, a.group * kQDim<PAIR> * ob, kRsrcFlags);
    f.rc = f.ra;
  } else {
    const int64_t slot0 = ((int64_t)w * 2 + k) * a.group;
    f.ra = __builtin_amdgcn_make_buffer_rsrc((void*)(a.ws_acc + slot0 * kHeadDim), (short)0,
                                             a.group * kHeadDim * 4, kRsrcFlags);
    f.rc = __builtin_amdgcn_make_buffer_rsrc((void*)(a.ws_ml + slot0 * 2), (short)0, a.group * 8,
                                             kRsrcFlags);
  }
}

template <bool PAIR>
MKV_DEV void finish_small_group(const DecodeArgs& a, const Cursor& c, bool whole, int w, int k,
                                const f32x4 (&acc)[8], float m_col, float l_col, float v_mul,
                                FinishStores& f) {
  const int lane = threadIdx.x & 63;
  // this lane's head after the spread, the lane holding its dims, its
  // register among acc[.][0..3], and the dims' offsets in the output row and
  // in the partial slots (head-major, 128 floats per head)
  int h, src, sel, out_off, part_off;
  if constexpr (PAIR) {
    h = lane >> 3;
    const int d = lane & 7;
    const bool hi = h >= (a.group >> 1);
    src = 16 * (h >> 2) + (hi ? 8 : 0) + d;
    sel = h & 3;
    out_off = h * kQDim<PAIR> + 8 * d;
    part_off = h * kHeadDim + (hi ? 64 : 0) + 8 * d;
  } else {
    h = lane >> 4;
    src = lane & 15;
    sel = h;
    out_off = h * kQDim<PAIR> + 8 * src;
    part_off = h * kHeadDim + 8 * src;
  }
  float x[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) {
    const float t0 = __shfl(acc[mm][0], src), t1 = __shfl(acc[mm][1], src);
    const float t2 = __shfl(acc[mm][2], src), t3 = __shfl(acc[mm][3], src);
    x[mm] = sel == 0 ? t0 : (sel == 1 ? t1 : (sel == 2 ? t2 : t3));
  }
  const float lh = __shfl(l_col, h);
  const float mh = __shfl(m_col, h);
  const bool valid = h < a.group;
  const bool first = PAIR ? (lane & 7) == 0 : (lane & 15) == 0;  // stores the head's (m, l)
  if (whole) {
    const float inv = lh > 0.0f ? v_mul / lh : 0.0f;
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) x[mm] *= inv;
    const int ob = a.q_dtype == MKV_DTYPE_F32 ? 4 : 2;
    finish_rsrc<PAIR>(a, true, c.b, c.kvh, w, k, f);
    const uint32_t off = (uint32_t)(out_off * ob);
    if (a.q_dtype == MKV_DTYPE_F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f.da[j] = __float_as_uint(x[j]);
        f.db[j] = __float_as_uint(x[4 + j]);
      }
      f.oa = valid ? off : kOob;
      f.ob = valid ? off + 16 : kOob;
    } else {
      const bool bf = a.q_dtype == MKV_DTYPE_BF16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = bf ? f32_to_bf16_bits(x[2 * j]) : f32_to_f16_bits(x[2 * j]);
        const uint32_t hi = bf ? f32_to_bf16_bits(x[2 * j + 1]) : f32_to_f16_bits(x[2 * j + 1]);
        f.da[j] = lo | (hi << 16);
      }
      f.oa = valid ? off : kOob;
      f.ob = kOob;
    }
    f.oc = kOob;
  } else {
    // (with pairing only the head's own half of its 128-float slot is
    // written; the merge kernel stores only that half)
    finish_rsrc<PAIR>(a, false, c.b, c.kvh, w, k, f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f.da[j] = __float_as_uint(x[j]);
      f.db[j] = __float_as_uint(x[4 + j]);
    }
    const uint32_t off = (uint32_t)(part_off * 4);
    f.oa = valid ? off : kOob;
    f.ob = valid ? off + 16 : kOob;
    f.dc = u32x2{__float_as_uint(mh), __float_as_uint(lh)};
    f.oc = valid && first ? (uint32_t)(h * 8) : kOob;
  }
}

MKV_DEV void issue_finish(const FinishStores& f) {
  __builtin_amdgcn_raw_buffer_store_b128(f.da, f.ra, f.oa, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(f.db, f.ra, f.ob, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b64(f.dc, f.rc, f.oc, 0, 0);
}

// Per-sequence tile counts and their prefix into LDS (every workgroup does it;
// workgroup 0 also publishes them for the merge kernel).  Returns the total
// number of columns of the stream.
MKV_DEV int64_t stream_prefix(const DecodeArgs& a, int* pre, int* lens) {
  __shared__ int wave_tot[kDecWaves];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  int running = 0;
  for (int base = 0; base < a.batch; base += kDecWaves * kWave) {
    const int b = base + tid;
    int n = 0;
    if (b < a.batch) {
      int64_t L = load_index(a.context_lens, b, a.ctx_i64);
      L = L < 0 ? 0 : (L > cap ? cap : L);
      lens[b] = (int)L;
      n = (int)((L + kTileTok - 1) / kTileTok);
    }
    // inclusive scan inside the wave (shuffles), then across the waves
    int incl = n;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_up(incl, off);
      incl += lane >= off ? y : 0;
    }
    if (lane == kWave - 1) wave_tot[wv] = incl;
    __syncthreads();
    int before = running, total = running;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const int t = wave_tot[w];
      before += w < wv ? t : 0;
      total += t;
    }
    if (b < a.batch) pre[b + 1] = before + incl;
    running = total;
    __syncthreads();
  }
  if (tid == 0) pre[0] = 0;
  __syncthreads();
  return running;
}

// Static split of the T columns of the stream over the W / Hkv wave groups:
// group w runs the contiguous range [begin(w), end(w)).  When two workgroups
// share each CU, the two waves on a SIMD do not progress at the same rate:
// issue arbitration favours the older wave, i.e. the one whose workgroup was
// dispatched in the first round (workgroups 0 .. CUs-1).  The groups of those
// waves (w1 of them) therefore get kFirstSharePct percent of the columns and
// the second-round groups the rest; with one workgroup per CU the split is
// even (w1 = W / Hkv).
// (Batch-256 FP8 step with the reversed head order below, against 58: 60
// +0.3%, 62 -1.5%; per-wave timestamps at 58 had the second-round groups
// end ~2.6 us after the first-round ones.)
constexpr int kFirstSharePct = 60;
// Split units per column (the cost-balanced split below).  Every range is at
// least kColCost units wide, so a range inside an item holds at least one of
// its columns: the merge kernel reads every group between an item's first and
// last contributor.
constexpr int kColCost = 4;
// Split units for entering a sequence: 1.25 columns (against 0, 0.75 and 2
// columns: +0.9% at the batch-256 FP8 step, +1-4% at batches 8-128).
constexpr int kSeqCost = 5;

// Contiguous split of `total` units (columns) over `parts` parts (wave
// groups); the first `parts1` parts (the first dispatch round) take
// kFirstSharePct percent of the units.
struct StreamSplit {
  int64_t total;
  int64_t base;  // units of the first-round parts
  int64_t per1, per2;
  int parts1, parts;

  MKV_DEV int64_t begin(int p) const {
    const int64_t b = p < parts1 ? (int64_t)p * per1 : base + (int64_t)(p - parts1) * per2;
    const int64_t cap = p < parts1 ? base : total;
    return b < cap ? b : cap;
  }
  MKV_DEV int64_t end(int p) const {
    const int64_t e = p < parts1 ? (int64_t)(p + 1) * per1 : base + (int64_t)(p - parts1 + 1) * per2;
    const int64_t cap = p < parts1 ? base : total;
    return e < cap ? e : cap;
  }
  // the part whose range holds unit g
  MKV_DEV int part_of(int64_t g) const {
    return g < base ? (int)(g / per1) : parts1 + (int)((g - base) / per2);
  }
};

MKV_DEV StreamSplit make_split(int64_t total, int parts, int first_parts, int first_pct) {
  StreamSplit p;
  p.total = total;
  p.parts = parts;
  if (first_parts <= 0 || first_parts >= parts) {
    p.parts1 = parts;
    p.per1 = (total + parts - 1) / parts;
    p.per1 = p.per1 < kColCost ? kColCost : p.per1;
    p.base = total;
    p.per2 = 1;
    return p;
  }
  p.parts1 = first_parts;
  const int64_t t1 = total * first_pct / 100;
  p.per1 = (t1 + first_parts - 1) / first_parts;
  p.per1 = p.per1 < kColCost ? kColCost : p.per1;
  const int64_t head = (int64_t)first_parts * p.per1;
  p.base = head < total ? head : total;
  const int p2 = parts - first_parts;
  p.per2 = (total - p.base + p2 - 1) / p2;
  p.per2 = p.per2 < kColCost ? kColCost : p.per2;
  return p;
}

// The group split of a launch: groups of Hkv consecutive waves (waves past
// the last whole group stay idle).
MKV_DEV StreamSplit stream_split(const DecodeArgs& a, int64_t columns) {
  const int groups = a.num_waves / a.num_kv_heads;
  const int first = a.first_waves >= a.num_waves ? groups : a.first_waves / a.num_kv_heads;
  return make_split(columns, groups, first, a.first_pct);
}

// Cost-balanced split.  A wave's time is its tiles plus a fixed cost for
// every sequence its range enters (the item's q, its finish stores and its
// partial last tile: ~1.25 tiles measured per sequence), so the groups split
// a cost stream, not the column stream: column g of sequence b costs
// kColCost units and stands at cost(g) = kColCost * g + a.seq_cost * b
// (kColCost is defined with the split above).

MKV_DEV int64_t stream_cost_total(const DecodeArgs& a, int64_t columns) {
  return kColCost * columns + (int64_t)a.seq_cost * a.batch;
}


// The sequences holding the costs x0 and x1 (<= the stream's total): the
// largest b < B with cost(b) = kColCost * pre[b] + seq_cost * b <= x, found
// lane-parallel (64 sequences per LDS read, one ballot each; b = 0 always
// qualifies), where a binary search took a chain of dependent LDS reads.
MKV_DEV void cost_seqs(const DecodeArgs& a, const int* pre, int64_t x0, int64_t x1, int& b0, int& b1) {
  const int lane = threadIdx.x & 63;
  int n0 = 0, n1 = 0;
  for (int j0 = 0; j0 < a.batch; j0 += kWave) {
    const int j = j0 + lane;
    bool c0 = false, c1 = false;
    if (j < a.batch) {
      const int64_t cj = kColCost * (int64_t)pre[j] + (int64_t)a.seq_cost * j;
      c0 = cj <= x0;
      c1 = cj <= x1;
    }
    n0 += __builtin_popcountll(__builtin_amdgcn_ballot_w64(c0));
    n1 += __builtin_popcountll(__builtin_amdgcn_ballot_w64(c1));
  }
  b0 = n0 - 1;
  b1 = n1 - 1;
}

// The first column of sequence b (from cost_seqs) whose cost is at least x;
// the sequence's column count past its end.
MKV_DEV int64_t cost_col_in_seq(const DecodeArgs& a, const int* pre, int b, int64_t x) {
  const int64_t p0 = lds_uniform(pre, b), p1 = lds_uniform(pre, b + 1);
  const int64_t rem = x - kColCost * p0 - (int64_t)a.seq_cost * b;
  const int64_t g = p0 + (rem <= 0 ? 0 : (rem + kColCost - 1) / kColCost);
  return g < p1 ? g : p1;
}

// The tile of KV head kvh at column g (g < pre[B]): sequence b is the largest
// b < B with pre[b] <= g (it has tiles), found lane-parallel as in cost_seqs.
MKV_DEV Cursor cursor_at_par(const int* pre, const int* lens, int B, int kvh, int64_t g) {
  const int lane = threadIdx.x & 63;
  int n = 0;
  for (int j0 = 0; j0 < B; j0 += kWave) {
    const int j = j0 + lane;
    n += __builtin_popcountll(__builtin_amdgcn_ballot_w64(j < B && pre[j] <= g));
  }
  const int b = n - 1;
  Cursor c;
  c.b = b;
  c.kvh = kvh;
  const int p0 = lds_uniform(pre, b);
  c.n = lds_uniform(pre, b + 1) - p0;
  c.t = (int)(g - p0);
  c.L = lds_uniform(lens, b);
  return c;
}

// Workgroup 0 publishes, per sequence, the groups whose ranges hold its
// first and last columns and the partial slot the first of them used (0 when
// its range starts exactly at the sequence), for the merge kernel.  (Spread
// over the grid, one sequence per workgroup, it delayed the first wave of
// every workgroup instead of one workgroup: the step ran 0.3% slower.)
MKV_DEV void publish_merge_meta(const DecodeArgs& a, const StreamSplit& sp, const int* pre) {
  int* meta = a.sk_meta + a.batch + 1;
  for (int b = threadIdx.x; b < a.batch; b += blockDim.x) {
    const int64_t p0 = pre[b], p1 = pre[b + 1];
    int glo = 0, ghi = 0, s0 = 0;
    if (p1 > p0) {
      const int64_t base = (int64_t)a.seq_cost * b;
      glo = sp.part_of(kColCost * p0 + base);
      ghi = sp.part_of(kColCost * (p1 - 1) + base);
      // first column of glo's range, by the same rule as cost_col_in_seq
      const int64_t x = sp.begin(glo);
      int lo = 0, hi = a.batch;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (kColCost * (int64_t)pre[mid] + (int64_t)a.seq_cost * mid <= x) lo = mid; else hi = mid;
      }
      const int64_t q0 = pre[lo], q1 = pre[lo + 1];
      const int64_t rem = x - kColCost * q0 - (int64_t)a.seq_cost * lo;
      int64_t g0 = q0 + (rem <= 0 ? 0 : (rem + kColCost - 1) / kColCost);
      g0 = g0 < q1 ? g0 : q1;
      s0 = p0 <= g0 ? 0 : 1;
    }
    meta[3 * b] = glo;
    meta[3 * b + 1] = ghi;
    meta[3 * b + 2] = s0;
  }
  for (int i = threadIdx.x; i <= a.batch; i += blockDim.x) a.sk_meta[i] = pre[i];
}

// KV head of wave slot k of a stream-K group (k = w % Hkv), and the slot of
// KV head kvh: reversed.  With 8 KV heads a group is two workgroups, which
// the dispatcher puts on neighbouring XCDs; the identity (first workgroup:
// heads 0-3, the first half of every 1 KB token row) left that workgroup's
// waves ~2.5% behind the other's on every group (per-wave timestamps), and
// every other order measured (reversed, halves swapped, interleaved) ran
// the batch-256 FP8 step 1.1% faster (6302 -> 6373-6380 GB/s, three A/B
// repeats in one call).
MKV_DEV int sk_head(int k, int hkv) { return hkv - 1 - k; }
MKV_DEV int sk_slot(int kvh, int hkv) { return hkv - 1 - kvh; }

template <int KV_DT, bool kSmallGroup, bool PAIR>
MKV_DEV void stream_decode(const DecodeArgs& a) {
  constexpr int kEb = DTypeInfo<KV_DT>::kBytes;
  extern __shared__ int sk_lds[];
  int* pre = sk_lds;                 // [batch + 1]
  int* lens = sk_lds + a.batch + 1;  // [batch]
  // deferred finishes of this wave: a.defer records of 64 lanes x 64 bytes,
  // then 4 ints each (whole, sequence, KV head, slot)
  const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  u32x4* dq = reinterpret_cast<u32x4*>(sk_lds + ((2 * a.batch + 1 + 3) & ~3)) + wl * a.defer * kWave * 4;
  int* dqu = reinterpret_cast<int*>(reinterpret_cast<u32x4*>(sk_lds + ((2 * a.batch + 1 + 3) & ~3)) +
                                    kDecWaves * a.defer * kWave * 4) + wl * a.defer * 4;
  int ndef = 0;
  const StreamSplit sp = stream_split(a, stream_cost_total(a, stream_prefix(a, pre, lens)));
  // Workgroup 0's waves publish the merge metadata when they leave (each
  // lane its own sequences; pre stays in LDS), not before their first tile.
  auto leave = [&]() {
    if (blockIdx.x == 0) publish_merge_meta(a, sp, pre);
  };

  const int lane = threadIdx.x & 63;
  const int c = lane & 15, kg = lane >> 4;
  const int w = blockIdx.x * kDecWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = w / a.num_kv_heads;  // this wave: KV head w % Hkv of its group's columns
  const int kvh = sk_head(w - grp * a.num_kv_heads, a.num_kv_heads);
  if (grp >= sp.parts) return leave();
  int64_t g0, g1;
  {
    const int64_t x0 = sp.begin(grp), x1 = sp.end(grp);
    int b0, b1;
    cost_seqs(a, pre, x0, x1, b0, b1);
    g0 = cost_col_in_seq(a, pre, b0, x0);
    g1 = cost_col_in_seq(a, pre, b1, x1);
  }
  if (g0 >= g1) return leave();

  const int row_bytes = (int)(a.idx.row_elems * kEb);
  const int64_t blk_bytes = (int64_t)row_bytes << a.idx.bs_log2;
  const int k_voff = c * row_bytes + 32 * kg * kEb;
  const int v_voff = 4 * kg * row_bytes + 8 * c * kEb;
  const float v_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.v_scale) : 1.0f;
  const float k_mul = (KV_DT == MKV_DTYPE_FP8E4M3) ? load_uniform_f32(a.k_scale) : 1.0f;
  const bool hi = PAIR && c >= (a.group >> 1);

  Cursor cc = cursor_at_par(pre, lens, a.batch, kvh, g0);  // tile being computed
  Cursor lc = cc;                                                  // next tile to load
  int64_t lg = g0;                                                 // its global index
  PhysPair ph_next;
  // Advance the load cursor; tiles past this wave's range are loaded as empty
  // (L = 0: no bytes move), selected without a branch so that the load
  // stream stays unconditional and the wait-count pass never drains it.
  auto advance_load = [&]() {
    cursor_next(lc, pre, lens, a.batch);
    ++lg;
    lc.L = lg < g1 ? lc.L : 0;
    ph_next = tile_phys(a, lc);
  };
  // Two register tiles: while tile g is computed, tile g+1 is in flight.  Two
  // waves share each SIMD (three tiles would push the FP8 kernel past the 256
  // registers that allow it), so each SIMD still has two tiles in flight.
  Tile16<KV_DT> t0b, t1b;
  // q of the item whose tile was issued last (16-bit q; an fp32 q is loaded
  // when its item starts).
  QStage qs;
  const bool q16 = a.q_dtype != MKV_DTYPE_F32;
  ph_next = tile_phys(a, lc);
  load_tile_sk<KV_DT, PAIR>(a, lc, ph_next, row_bytes, blk_bytes, k_voff, v_voff, t0b);
  load_q_stage<PAIR>(a, lc.b, lc.kvh, true, qs);
  advance_load();

  QOps<KV_DT> qop;
  float score_mul = 0.0f;
  f32x4 acc[8];
  float m_run = kNegBig, l_run = 0.0f;
  int64_t item_g0 = g0 - cc.t;  // column of the current item's first tile

  // One pipeline step: prefetch tile g+1 into `nxt`, compute tile g in `cur`.
  auto step = [&](Tile16<KV_DT>& cur, Tile16<KV_DT>& nxt, int64_t g) {
    load_tile_sk<KV_DT, PAIR>(a, lc, ph_next, row_bytes, blk_bytes, k_voff, v_voff, nxt);
    if (cc.t == 0 || g == g0) {  // a new item starts: its q, fresh softmax state
      score_mul = q16 ? staged_q_operands<KV_DT>(a, qs, qop, k_mul)
                      : load_q_operands<KV_DT, PAIR>(a, cc.b, cc.kvh, qop, k_mul);
#pragma unroll
      for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_run = kNegBig;
      l_run = 0.0f;
      item_g0 = g - cc.t;
    }
    // q of the item that the tile just issued starts (an empty load otherwise)
    load_q_stage<PAIR>(a, lc.b, lc.kvh, lc.t == 0, qs);
    advance_load();
    compute_tile16<KV_DT, PAIR>(cur, cc.t * kTileTok, cc.L, qop, score_mul, acc, m_run, l_run, hi);
    const bool item_end = cc.t == cc.n - 1;
    const bool fin = item_end || g == g1 - 1;
    const bool whole = item_end && item_g0 >= g0;
    const int kslot = item_g0 <= g0 ? 0 : 1;
    if constexpr (kSmallGroup) {
      FinishStores fs;
      finish_none(fs);
      if (fin) {
        float l_col = l_run + __shfl_xor(l_run, 16);
        l_col += __shfl_xor(l_col, 32);
        finish_small_group<PAIR>(a, cc, whole, w, kslot, acc, m_run, l_col, v_mul, fs);
        // Finishes before the range's last tile wait in LDS (up to
        // a.defer of them) and go out after it, so that their stores do not
        // sit between the tile loads of the read stream.
        if (g != g1 - 1 && ndef < a.defer) {
          u32x4* rec = dq + (ndef * kWave + lane) * 4;
          rec[0] = fs.da;
          rec[1] = fs.db;
          rec[2] = u32x4{fs.dc[0], fs.dc[1], fs.oa, fs.ob};
          rec[3] = u32x4{fs.oc, 0u, 0u, 0u};
          if (lane == 0) {
            int* u = dqu + 4 * ndef;
            u[0] = whole ? 1 : 0;
            u[1] = cc.b;
            u[2] = cc.kvh;
            u[3] = kslot;
          }
          ++ndef;
          finish_none(fs);
        }
      }
      issue_finish(fs);
    } else if (fin) {
      float l_col = l_run + __shfl_xor(l_run, 16);
      l_col += __shfl_xor(l_col, 32);
      finish_sk<PAIR>(a, cc, whole, w, kslot, acc, m_run, l_col, v_mul);
    }
    cursor_next(cc, pre, lens, a.batch);
  };
  for (int64_t g = g0;;) {
    step(t0b, t1b, g);
    if (++g >= g1) break;
    step(t1b, t0b, g);
    if (++g >= g1) break;
  }
  if constexpr (kSmallGroup) {
    for (int i = 0; i < ndef; ++i) {
      const int* u = dqu + 4 * i;
      FinishStores fs;
      finish_rsrc<PAIR>(a, lds_uniform(u, 0) != 0, lds_uniform(u, 1), lds_uniform(u, 2), w, lds_uniform(u, 3),
                        fs);
      const u32x4* rec = dq + (i * kWave + lane) * 4;
      fs.da = rec[0];
      fs.db = rec[1];
      const u32x4 r2 = rec[2];
      fs.dc = u32x2{r2[0], r2[1]};
      fs.oa = r2[2];
      fs.ob = r2[3];
      fs.oc = rec[3][0];
      issue_finish(fs);
    }
  }
  leave();
}

template <int KV_DT, bool kSmallGroup, bool PAIR>
__global__ __launch_bounds__(kDecWaves* kWave) void paged_decode_stream_kernel(DecodeArgs a) {
  stream_decode<KV_DT, kSmallGroup, PAIR>(a);
}

// Per-token-head formats (and per-tensor FP8 with groups above 4) ask for
// the two-waves-per-SIMD register budget explicitly: left to itself the
// scheduler takes a few registers more than two waves can hold, and the
// residency halves.
template <int KV_DT, bool kSmallGroup, bool PAIR>
__global__ __launch_bounds__(kDecWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void
paged_decode_stream_2w_kernel(DecodeArgs a) {
  stream_decode<KV_DT, kSmallGroup, PAIR>(a);
}

template <int KV_DT, bool kSmallGroup, bool PAIR>
constexpr auto stream_kernel() {
  // (per-tensor FP8 with groups above 4 lands a few registers past 256 on its own)
  if constexpr (kPerTokenScale<KV_DT> || (KV_DT == MKV_DTYPE_FP8E4M3 && !kSmallGroup))
    return paged_decode_stream_2w_kernel<KV_DT, kSmallGroup, PAIR>;
  else
    return paged_decode_stream_kernel<KV_DT, kSmallGroup, PAIR>;
}

// Element offset, inside the batch row, of the two output dims 2 lane and
// 2 lane + 1 of query head hq (head h of its group) that a merge wave's lane
// writes; own = false when they belong to the other half of a paired head.
MKV_DEV int64_t merge_out_offset(const DecodeArgs& a, int hq, int h, int lane, bool& own) {
  if (!a.pair) {
    own = true;
    return (int64_t)hq * kHeadDim + 2 * lane;
  }
  const bool hi = h >= (a.group >> 1);
  own = (lane >= 32) == hi;
  return (int64_t)hq * (kHeadDim / 2) + 2 * lane - (hi ? 64 : 0);
}

MKV_DEV void store_out2(const DecodeArgs& a, int64_t off, float x0, float x1) {
  if (a.q_dtype == MKV_DTYPE_F32) {
    *reinterpret_cast<f32x2*>(reinterpret_cast<float*>(a.out) + off) = f32x2{x0, x1};
  } else {
    const uint32_t lo = a.q_dtype == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x0) : f32_to_f16_bits(x0);
    const uint32_t hi = a.q_dtype == MKV_DTYPE_BF16 ? f32_to_bf16_bits(x1) : f32_to_f16_bits(x1);
    *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.out) + off) = lo | (hi << 16);
  }
}

// Merge of stream-K partials: one wave per (sequence, query head).  The
// partials of an item (sequence, KV head kvh) come from wave kvh of the
// consecutive groups glo..ghi, one slot each.
// Lane i reads (m, l) of contributor wlo + i, so the maximum and the
// denominator are wave reductions rather than a chain of dependent loads, and
// the accumulator rows are read four contributors at a time (independent
// loads in flight) with each contributor's weight taken from its lane.
MKV_DEV int merge_slot(const DecodeArgs& a, int glo, int s0, int grp, int kvh, int h) {
  const int wp = grp * a.num_kv_heads + sk_slot(kvh, a.num_kv_heads);
  return ((wp * 2 + (grp == glo ? s0 : 0)) * a.group + h);
}

__global__ __launch_bounds__(kDecWaves* kWave) void paged_decode_stream_merge_kernel(DecodeArgs a,
                                                                                     int kv_fp8) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = (int64_t)blockIdx.x * kDecWaves + (threadIdx.x >> 6);
  if (wv >= (int64_t)a.batch * a.num_heads) return;
  const int b = (int)(wv / a.num_heads);
  const int hq = (int)(wv - (int64_t)b * a.num_heads);
  const int kvh = hq / a.group, h = hq - kvh * a.group;
  const int p0 = a.sk_meta[b], n = a.sk_meta[b + 1] - p0;
  const int* meta = a.sk_meta + a.batch + 1 + 3 * b;
  bool own;
  const int64_t off = (int64_t)b * a.out_stride + merge_out_offset(a, hq, h, lane, own);
  float o0 = 0.0f, o1 = 0.0f, l = 0.0f;
  if (n > 0) {
    const int glo = meta[0], ghi = meta[1], s0 = meta[2];
    if (glo == ghi) return;  // written whole by the main kernel
    const int nc = ghi - glo + 1;
    if (nc <= kWave) {
      // One round trip for the common case: every contributor's (m, l),
      // lane-parallel, and the first four accumulator rows are loaded
      // together (the rows' slots do not depend on (m, l)); the weights
      // follow from the maximum, the remaining rows four at a time.
      const int my_slot = lane < nc ? merge_slot(a, glo, s0, glo + lane, kvh, h) : 0;
      f32x2 x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // nc >= 2; rows u >= nc repeat row 0 with weight 0
        const int64_t sl = __builtin_amdgcn_readlane(my_slot, u);
        x[u] = *reinterpret_cast<const f32x2*>(a.ws_acc + (u < nc ? sl : 0) * kHeadDim + 2 * lane);
      }
      const f32x2 ml = lane < nc ? *reinterpret_cast<const f32x2*>(a.ws_ml + (int64_t)my_slot * 2)
                                 : f32x2{kNegBig, 0.0f};
      const float M = wave_max(ml[0]);
      const float wgt = lane < nc ? __builtin_amdgcn_exp2f(ml[0] - M) : 0.0f;
      l = wgt * ml[1];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), u));
        o0 += w1 * x[u][0];
        o1 += w1 * x[u][1];
      }
      for (int j = 4; j < nc; j += 4) {
        f32x2 y[4];
        float w4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t sl = __builtin_amdgcn_readlane(my_slot, j + u < nc ? j + u : 0);
          w4[u] = j + u < nc ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j + u)) : 0.0f;
          y[u] = *reinterpret_cast<const f32x2*>(a.ws_acc + sl * kHeadDim + 2 * lane);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          o0 += w4[u] * y[u][0];
          o1 += w4[u] * y[u][1];
        }
      }
    } else {
      float M = kNegBig;
      for (int c0 = 0; c0 < nc; c0 += kWave) {
        if (c0 + lane < nc) M = fmaxf(M, a.ws_ml[(int64_t)merge_slot(a, glo, s0, glo + c0 + lane, kvh, h) * 2]);
      }
      M = wave_max(M);
      for (int c0 = 0; c0 < nc; c0 += kWave) {
        int my_slot = 0;
        float wgt = 0.0f;
        if (c0 + lane < nc) {
          my_slot = merge_slot(a, glo, s0, glo + c0 + lane, kvh, h);
          wgt = __builtin_amdgcn_exp2f(a.ws_ml[(int64_t)my_slot * 2] - M);
          l += wgt * a.ws_ml[(int64_t)my_slot * 2 + 1];
        }
        const int cnt = nc - c0 < kWave ? nc - c0 : kWave;
        int j = 0;
        for (; j + 4 <= cnt; j += 4) {
          f32x2 x[4];
          float w4[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int64_t sl = __builtin_amdgcn_readlane(my_slot, j + u);
            w4[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j + u));
            x[u] = *reinterpret_cast<const f32x2*>(a.ws_acc + sl * kHeadDim + 2 * lane);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            o0 += w4[u] * x[u][0];
            o1 += w4[u] * x[u][1];
          }
        }
        for (; j < cnt; ++j) {
          const int64_t sl = __builtin_amdgcn_readlane(my_slot, j);
          const float w1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), j));
          const f32x2 x = *reinterpret_cast<const f32x2*>(a.ws_acc + sl * kHeadDim + 2 * lane);
          o0 += w1 * x[0];
          o1 += w1 * x[1];
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
  }
  const float inv = l > 0.0f ? (kv_fp8 ? load_uniform_f32(a.v_scale) : 1.0f) / l : 0.0f;
  if (own) store_out2(a, off, o0 * inv, o1 * inv);
}

// ---------------------------------------------------------------------------
// fp32 KV kernel: v_mfma_f32_16x16x4_f32, 16-token tiles, same lane mapping.
// ---------------------------------------------------------------------------
template <bool PAIR>
__global__ __launch_bounds__(kDecWaves* kWave) void paged_decode_mfma32_kernel(DecodeArgs a) {
  WorkItem it;
  if (!decode_work_item(a, wave_work_index(), it)) return;
  float qf[32];
  load_q_f32<PAIR>(a, it.b, it.kvh, qf);
  const float score_mul = a.sm_scale * kLog2e;
  f32x4 acc[8];
#pragma unroll
  for (int mm = 0; mm < 8; ++mm) acc[mm] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig, l_run = 0.0f;
  f32_range(a, it, qf, score_mul, acc, m_run, l_run);
  float l_col = l_run + __shfl_xor(l_run, 16);
  l_col += __shfl_xor(l_col, 32);
  finish_item<PAIR>(a, it, acc, m_run, l_col, 1.0f);
}

// ---------------------------------------------------------------------------
// Split-K merge: one wave per (b, query head) whose sequence used > 1 split.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kDecWaves* kWave) void paged_decode_merge_kernel(DecodeArgs a,
                                                                              int kv_fp8) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * kDecWaves + (threadIdx.x >> 6);
  if (w >= (int64_t)a.batch * a.num_heads) return;
  const int b = (int)(w / a.num_heads);
  const int hq = (int)(w - (int64_t)b * a.num_heads);
  int64_t L = load_index(a.context_lens, b, a.ctx_i64);
  const int64_t cap = (int64_t)a.idx.max_blocks << a.idx.bs_log2;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  const int ns = L > 0 ? (int)((L + a.split_tokens - 1) / a.split_tokens) : 1;
  if (ns <= 1) return;
  const int64_t slot0 = ((int64_t)b * a.num_heads + hq) * a.max_splits;
  float M = kNegBig;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, a.ws_ml[(slot0 + s) * 2]);
  float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < ns; ++s) {
    const float wgt = __builtin_amdgcn_exp2f(a.ws_ml[(slot0 + s) * 2] - M);
    l += wgt * a.ws_ml[(slot0 + s) * 2 + 1];
    const f32x2 x = *reinterpret_cast<const f32x2*>(a.ws_acc + (slot0 + s) * kHeadDim + 2 * lane);
    o0 += wgt * x[0];
    o1 += wgt * x[1];
  }
  const float inv = l > 0.0f ? (kv_fp8 ? load_uniform_f32(a.v_scale) : 1.0f) / l : 0.0f;
  bool own;
  const int64_t off = (int64_t)b * a.out_stride + merge_out_offset(a, hq, hq % a.group, lane, own);
  if (own) store_out2(a, off, o0 * inv, o1 * inv);
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

int default_split_tokens(int batch, int num_kv_heads, int max_blocks, int block_size) {
  // Aim for >= ~4096 work items (256 CUs x 16 waves) so that the grid fills
  // the chip even when the batch is small, but never split below 64 tokens.
  const int64_t items = (int64_t)batch * num_kv_heads;
  const int64_t max_len = (int64_t)max_blocks * block_size;
  int64_t want_splits = (4096 + items - 1) / (items > 0 ? items : 1);
  int64_t st = (max_len + want_splits - 1) / (want_splits > 0 ? want_splits : 1);
  st = ((st + 31) / 32) * 32;
  if (st < 64) st = 64;
  if (st > 512) st = 512;
  return (int)st;
}

int resolve_split(int split_tokens, int batch, int num_kv_heads, int max_blocks, int block_size) {
  if (split_tokens <= 0) return default_split_tokens(batch, num_kv_heads, max_blocks, block_size);
  return split_tokens;
}

// The three decode schedules (mkv_paged_decode_route reports them).
constexpr int kRouteStream = MKV_DECODE_ROUTE_STREAM;
constexpr int kRouteSplit = MKV_DECODE_ROUTE_SPLIT;
constexpr int kRouteWorkgroup = MKV_DECODE_ROUTE_WORKGROUP;

// Compute units of the current device (cached per device).  Without a usable
// device the size query assumes a generous count; no kernel runs then.
int device_cus() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 512;
    cache[dev] = n;
  }
  return cache[dev];
}

// Persistent stream-K grid: at most two 4-wave workgroups per CU (two waves
// per SIMD); the launch uses what the kernel's register budget allows.
constexpr int kStreamWgPerCu = 2;

template <typename K>
int resident_wgs_per_cu(K kernel, size_t lds) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kDecWaves * kWave, lds) != hipSuccess || n < 1)
    n = 1;
  return n < kStreamWgPerCu ? n : kStreamWgPerCu;
}

int stream_waves() { return device_cus() * kStreamWgPerCu * kDecWaves; }

size_t stream_ws_bytes(int batch, int group) {
  const size_t w = (size_t)stream_waves();
  return w * 2 * group * (kHeadDim + 2) * sizeof(float) + (size_t)(4 * batch + 2) * sizeof(int);
}

// Persistent stream-K launch: one wave per SIMD slot the kernel can hold
// (residency cached per device and LDS bucket), the first dispatch round
// marked for the uneven split.
template <int DT, bool SMALL, bool PAIR>
void launch_stream(DecodeArgs& a, int lds_bucket, size_t lds_bound, size_t lds, hipStream_t s) {
  static int per_cu[64][2][2];
  int dev = 0;
  (void)hipGetDevice(&dev);
  const int slot = dev >= 0 && dev < 64 ? dev : 0;
  constexpr auto kernel = stream_kernel<DT, SMALL, PAIR>();
  int& res = per_cu[slot][lds_bucket][PAIR ? 1 : 0];
  if (res == 0) res = resident_wgs_per_cu(kernel, lds_bound);
  const int wgs = device_cus() * res;
  a.num_waves = wgs * kDecWaves;
  a.first_waves = res > 1 ? device_cus() * kDecWaves : a.num_waves;
  hipLaunchKernelGGL(kernel, dim3(wgs), dim3(kDecWaves * kWave), lds, s, a);
}

size_t split_ws_bytes(int batch, int num_heads, int max_blocks, int block_size, int st) {
  const int64_t max_splits = ((int64_t)max_blocks * block_size + st - 1) / st;
  if (max_splits <= 1) return 0;
  return (size_t)batch * num_heads * max_splits * (kHeadDim + 2) * sizeof(float);
}

// Kernel shape of a call: its KV heads and group as the kernels see them
// (head_dim 64: KV heads read in pairs, see kQDim).
struct KernelShape {
  int kv_heads;
  int group;
  bool pair;
};

// MKV_OK, or the status of a shape the kernels do not support.
int kernel_shape(int num_heads, int num_kv_heads, int head_dim, KernelShape& ks) {
  if (num_heads <= 0 || num_kv_heads <= 0) return MKV_ERR_BAD_SHAPE;
  if (head_dim != kHeadDim && head_dim != kHeadDim / 2) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  if (num_heads % num_kv_heads) return MKV_ERR_UNSUPPORTED_GROUP;
  const int g = num_heads / num_kv_heads;
  ks.pair = head_dim == kHeadDim / 2;
  if (ks.pair) {
    if (num_kv_heads & 1) return MKV_ERR_UNSUPPORTED_HEAD_DIM;  // heads pair up
    if (g > 8) return MKV_ERR_UNSUPPORTED_GROUP;                // 2g query heads per pair
    ks.kv_heads = num_kv_heads / 2;
    ks.group = 2 * g;
  } else {
    if (g > 16) return MKV_ERR_UNSUPPORTED_GROUP;
    ks.kv_heads = num_kv_heads;
    ks.group = g;
  }
  return MKV_OK;
}

// Waves per workgroup of the workgroup route: as many as fill the chip's
// wave slots once (a CU holds max_waves waves of the kernel: 8 at two waves
// per SIMD, 4 for the split-q kernel at one), no more than the widest
// sequence's tiles, and few enough that the LDS merge buffers fit in 64 KiB.
int wg_waves(int batch, int kv_heads, int group, int max_blocks, int block_size, int cus,
             int max_waves = kWgMaxWaves) {
  const int64_t items = (int64_t)batch * kv_heads;
  const int64_t slots = (int64_t)cus * max_waves;
  const int64_t max_tiles = ((int64_t)max_blocks * block_size + 31) / 32;
  int nw = max_waves;
  while (nw > 1 && (items * nw > slots || nw > max_tiles ||
                    (size_t)nw * group * (kHeadDim + 2) * sizeof(float) > 65536))
    nw >>= 1;
  return nw;
}

// The route of a call.  split_tokens > 0: split-K with that split;
// MKV_DECODE_WORKGROUP: the workgroup route; MKV_DECODE_STREAM: stream-K
// (split-K where stream-K does not apply: fp32 caches, batches above
// kStreamMaxBatch).  0, the library's choice, from the shape alone, with the
// block-table width as the bound of the longest context (the reference's
// runner pads each decode step's tables to its longest sequence,
// model_runner.py:640-644):
//   * the workgroup route (one launch, no workspace, no partial round trip
//     through HBM) when the longest possible item gives each of its waves
//     at most 128 tokens, whatever the batch; or at most 256 tokens when
//     its waves also fill enough wave slots (items x waves >= 2 x CUs for
//     per-tensor FP8, 6 x CUs for 16-bit caches, whose tiles are twice the
//     bytes; per-token-head FP8 / INT8 never); fp32 caches: at most 512
//     tokens with items x waves >= 2 x CUs.  Its time is set by the longest item's
//     tile chain, so short contexts favour it and long ones do not.
//     Measured (graph replays, 8 KV heads, FP8 / bf16 / FP8 per-token-head):
//     batches 1 / 4 of 300-800 tokens in 4-block tables (128 tokens a wave)
//     9.1 / 10.5, 11.5 / 13.3, 11.6 / 15.4 us against 13.9 / 15.0, 13.8 /
//     14.9, 14.0 / 15.0 us for stream-K and its merge; batches 8 / 16 of
//     1024-2048 tokens in 8-block tables (256 tokens a wave) FP8 20.1 / 21.6
//     against 22.5 / 23.9 us, bf16 28.3 / 30.7 against 21.0 / 28.1 us, at
//     batch 32 bf16 38.3 against 41.4 us; FP8 batches 1 / 4 there 15.4 /
//     17.8 against 18.4 / 21.0 us, per-token-head FP8 22.2 / 27.8 against
//     18.3 / 20.9 us (batches 8-32 and 60 likewise: 26-36 against 23-31
//     us); batch 32 of 256-4096 tokens: 42.9 against 34.8 us.
//     per_token: the call's scales are per token and head (INT8 always);
//     mkv_paged_decode_route, which has no scale mode, reports per-tensor
//     FP8's route for an FP8 dtype, and mkv_paged_decode_workspace_size
//     sizes for the larger of the two;
//   * stream-K otherwise (16-bit / FP8 / INT8 caches): balanced over every
//     wave whatever the lengths, at the cost of a merge launch;
//   * split-K for fp32 caches otherwise (default split; the workgroup route
//     took 37.0 us against 21.0 us for fp32 batch 4 of 207-798 tokens).
int choose_route(int split_tokens, int kv_dtype, int batch, const KernelShape& ks, int max_blocks,
                 int block_size, int cus, bool per_token = false) {
  if (split_tokens == MKV_DECODE_WORKGROUP) return kRouteWorkgroup;
  if (split_tokens > 0) return kRouteSplit;
  const bool stream_ok =
      kv_dtype != MKV_DTYPE_F32 && batch <= kStreamMaxBatch && ks.kv_heads <= cus * kDecWaves;
  if (split_tokens == MKV_DECODE_STREAM) return stream_ok ? kRouteStream : kRouteSplit;
  const int64_t items = (int64_t)batch * ks.kv_heads;
  const int nw = wg_waves(batch, ks.kv_heads, ks.group, max_blocks, block_size, cus);
  const int64_t wave_tokens = ((int64_t)max_blocks * block_size + nw - 1) / nw;
  const int64_t fill = items * nw;
  bool wg;
  if (kv_dtype == MKV_DTYPE_F32)
    wg = fill >= 2 * (int64_t)cus && wave_tokens <= 16 * kTileTok;
  else if (wave_tokens <= 4 * kTileTok)
    wg = true;
  else if (per_token || kv_dtype == MKV_DTYPE_I8)
    wg = false;
  else if (kv_dtype == MKV_DTYPE_FP8E4M3)
    wg = fill >= 2 * (int64_t)cus && wave_tokens <= 8 * kTileTok;
  else
    wg = fill >= 6 * (int64_t)cus && wave_tokens <= 8 * kTileTok;
  if (wg) return kRouteWorkgroup;
  return stream_ok ? kRouteStream : kRouteSplit;
}

// Workspace bytes of a route.
size_t route_ws_bytes(int route, int batch, int num_heads, const KernelShape& ks, int max_blocks,
                      int block_size, int split_tokens) {
  if (route == kRouteWorkgroup) return 0;
  if (route == kRouteStream) return stream_ws_bytes(batch, ks.group);
  const int st = resolve_split(split_tokens, batch, ks.kv_heads, max_blocks, block_size);
  return split_ws_bytes(batch, num_heads, max_blocks, block_size, st);
}

}  // namespace
}  // namespace mkv

using namespace mkv;

extern "C" int mkv_paged_decode_split_tokens(int batch, int num_kv_heads, int max_blocks,
                                             int block_size, int split_tokens) {
  return resolve_split(split_tokens, batch, num_kv_heads, max_blocks, block_size);
}

extern "C" int mkv_paged_decode_route(int batch, int num_heads, int num_kv_heads, int max_blocks,
                                      int block_size, int head_dim, int kv_dtype, int split_tokens,
                                      int num_cus) {
  KernelShape ks;
  if (batch <= 0 || max_blocks <= 0 || block_size <= 0) return MKV_ERR_BAD_SHAPE;
  const int st = kernel_shape(num_heads, num_kv_heads, head_dim, ks);
  if (st != MKV_OK) return st;
  return choose_route(split_tokens, kv_dtype, batch, ks, max_blocks, block_size,
                      num_cus > 0 ? num_cus : device_cus());
}

extern "C" size_t mkv_paged_decode_workspace_size(int batch, int num_heads, int num_kv_heads,
                                                  int max_blocks, int block_size, int head_dim,
                                                  int kv_dtype, int split_tokens) {
  KernelShape ks;
  if (batch <= 0 || max_blocks <= 0 || block_size <= 0 ||
      kernel_shape(num_heads, num_kv_heads, head_dim, ks) != MKV_OK)
    return 0;
  const int cus = device_cus();
  const int route = choose_route(split_tokens, kv_dtype, batch, ks, max_blocks, block_size, cus);
  const size_t n = route_ws_bytes(route, batch, num_heads, ks, max_blocks, block_size, split_tokens);
  if (kv_dtype != MKV_DTYPE_FP8E4M3) return n;
  // (per-token-head FP8 scales may take another route)
  const int rt = choose_route(split_tokens, kv_dtype, batch, ks, max_blocks, block_size, cus, true);
  const size_t nt = route_ws_bytes(rt, batch, num_heads, ks, max_blocks, block_size, split_tokens);
  return n > nt ? n : nt;
}

namespace {

// Launch the kernels of `route` (arguments validated, a filled in except the
// route's own fields).
template <bool PAIR>
int launch_route(DecodeArgs& a, int route, int fmt, int split_tokens, int max_blocks, int block_size,
                 void* workspace, size_t workspace_bytes, hipStream_t s) {
  const int batch = a.batch, group = a.group;
  // the merge kernels apply the per-tensor V scale
  const bool fp8 = fmt == MKV_DTYPE_FP8E4M3;
  if (route == kRouteWorkgroup) {
    // bf16 MFMA formats with an fp32 / fp16 q: the split-q kernel
    const bool qsplit = (fmt == MKV_DTYPE_BF16 || fmt == kKvFp8PerToken || fmt == kKvI8PerToken) &&
                        a.q_dtype != MKV_DTYPE_BF16;
    const int nw = wg_waves(batch, a.num_kv_heads, group, max_blocks, block_size, device_cus(),
                            qsplit ? kWgSplitWaves : kWgMaxWaves);
    const size_t lds = (size_t)nw * group * (kHeadDim + 2) * sizeof(float);
    a.split_tokens = 0;
    a.max_splits = 0;
    a.ws_acc = nullptr;
    a.ws_ml = nullptr;
    const dim3 grid((unsigned)((int64_t)batch * a.num_kv_heads)), block(nw * kWave);
    if (qsplit) {
      switch (fmt) {
        case kKvFp8PerToken:
          hipLaunchKernelGGL((paged_decode_wg_qsplit_kernel<kKvFp8PerToken, PAIR>), grid, block, lds, s, a);
          break;
        case kKvI8PerToken:
          hipLaunchKernelGGL((paged_decode_wg_qsplit_kernel<kKvI8PerToken, PAIR>), grid, block, lds, s, a);
          break;
        default:
          hipLaunchKernelGGL((paged_decode_wg_qsplit_kernel<MKV_DTYPE_BF16, PAIR>), grid, block, lds, s, a);
          break;
      }
      return (int)hipGetLastError();
    }
    switch (fmt) {
      case MKV_DTYPE_F32:
        hipLaunchKernelGGL(paged_decode_wg_f32_kernel<PAIR>, grid, block, lds, s, a);
        break;
      case MKV_DTYPE_FP8E4M3:
        hipLaunchKernelGGL((paged_decode_wg_kernel<MKV_DTYPE_FP8E4M3, PAIR>), grid, block, lds, s, a);
        break;
      case kKvFp8PerToken:
        hipLaunchKernelGGL((paged_decode_wg_kernel<kKvFp8PerToken, PAIR>), grid, block, lds, s, a);
        break;
      case kKvI8PerToken:
        hipLaunchKernelGGL((paged_decode_wg_kernel<kKvI8PerToken, PAIR>), grid, block, lds, s, a);
        break;
      case MKV_DTYPE_BF16:
        hipLaunchKernelGGL((paged_decode_wg_kernel<MKV_DTYPE_BF16, PAIR>), grid, block, lds, s, a);
        break;
      default:
        hipLaunchKernelGGL((paged_decode_wg_kernel<MKV_DTYPE_F16, PAIR>), grid, block, lds, s, a);
        break;
    }
    return (int)hipGetLastError();
  }
  if (route == kRouteStream) {
    const size_t need = stream_ws_bytes(batch, group);
    if (!workspace) return MKV_ERR_NULL_POINTER;
    if (workspace_bytes < need) return MKV_ERR_WORKSPACE_TOO_SMALL;
    if (reinterpret_cast<uintptr_t>(workspace) & 15u) return MKV_ERR_MISALIGNED;
    // (held finishes: the kernels for groups of at most 4 query heads)
    const bool small = group <= (PAIR ? 8 : 4);  // finish_small_group's heads
    a.defer = batch <= kStreamDeferMaxBatch && small ? kStreamDefer : 0;

    const size_t lds = stream_lds_bytes(batch, a.defer);
    // Workspace slots are laid out for the largest grid (stream_waves()).
    const size_t slots = (size_t)stream_waves() * 2 * group;
    a.split_tokens = kTileTok;
    a.max_splits = 0;
    a.ws_acc = reinterpret_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + slots * kHeadDim;
    a.sk_meta = reinterpret_cast<int*>(a.ws_ml + slots * 2);
    a.seq_cost = kSeqCost;
    a.first_pct = kFirstSharePct;
    // Residency depends on the launch's LDS (the per-sequence prefix): query it
    // once per device for batches up to kStreamSmallBatch and once for larger.
    const int lds_bucket = batch <= kStreamSmallBatch ? 0 : 1;
    const size_t lds_bound = lds_bucket ? kStreamMaxLds : kStreamSmallLds;
    switch (fmt) {
      case MKV_DTYPE_FP8E4M3:
        small ? launch_stream<MKV_DTYPE_FP8E4M3, true, PAIR>(a, lds_bucket, lds_bound, lds, s)
              : launch_stream<MKV_DTYPE_FP8E4M3, false, PAIR>(a, lds_bucket, lds_bound, lds, s);
        break;
      case kKvFp8PerToken:
        small ? launch_stream<kKvFp8PerToken, true, PAIR>(a, lds_bucket, lds_bound, lds, s)
              : launch_stream<kKvFp8PerToken, false, PAIR>(a, lds_bucket, lds_bound, lds, s);
        break;
      case kKvI8PerToken:
        small ? launch_stream<kKvI8PerToken, true, PAIR>(a, lds_bucket, lds_bound, lds, s)
              : launch_stream<kKvI8PerToken, false, PAIR>(a, lds_bucket, lds_bound, lds, s);
        break;
      case MKV_DTYPE_BF16:
        small ? launch_stream<MKV_DTYPE_BF16, true, PAIR>(a, lds_bucket, lds_bound, lds, s)
              : launch_stream<MKV_DTYPE_BF16, false, PAIR>(a, lds_bucket, lds_bound, lds, s);
        break;
      default:
        small ? launch_stream<MKV_DTYPE_F16, true, PAIR>(a, lds_bucket, lds_bound, lds, s)
              : launch_stream<MKV_DTYPE_F16, false, PAIR>(a, lds_bucket, lds_bound, lds, s);
        break;
    }
    const int64_t mitems = (int64_t)batch * a.num_heads;
    hipLaunchKernelGGL(paged_decode_stream_merge_kernel,
                       dim3((unsigned)((mitems + kDecWaves - 1) / kDecWaves)), dim3(kDecWaves * kWave), 0,
                       s, a, (int)fp8);
    return (int)hipGetLastError();
  }

  const int st = resolve_split(split_tokens, batch, a.num_kv_heads, max_blocks, block_size);
  a.split_tokens = st;
  const int64_t max_len = (int64_t)max_blocks * block_size;
  a.max_splits = max_len > 0 ? (int)((max_len + st - 1) / st) : 1;
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  if (a.max_splits > 1) {
    const size_t need = (size_t)batch * a.num_heads * a.max_splits * (kHeadDim + 2) * sizeof(float);
    if (!workspace) return MKV_ERR_NULL_POINTER;
    if (workspace_bytes < need) return MKV_ERR_WORKSPACE_TOO_SMALL;
    if (reinterpret_cast<uintptr_t>(workspace) & 15u) return MKV_ERR_MISALIGNED;
    a.ws_acc = reinterpret_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + (size_t)batch * a.num_heads * a.max_splits * kHeadDim;
  }
  const int64_t items = (int64_t)batch * a.num_kv_heads * a.max_splits;
  const dim3 grid((unsigned)((items + kDecWaves - 1) / kDecWaves));
  const dim3 block(kDecWaves * kWave);
  switch (fmt) {
    case MKV_DTYPE_FP8E4M3:
      hipLaunchKernelGGL((paged_decode_mfma16_kernel<MKV_DTYPE_FP8E4M3, PAIR>), grid, block, 0, s, a);
      break;
    case kKvFp8PerToken:
      hipLaunchKernelGGL((paged_decode_mfma16_2w_kernel<kKvFp8PerToken, PAIR>), grid, block, 0, s, a);
      break;
    case kKvI8PerToken:
      hipLaunchKernelGGL((paged_decode_mfma16_2w_kernel<kKvI8PerToken, PAIR>), grid, block, 0, s, a);
      break;
    case MKV_DTYPE_BF16:
      hipLaunchKernelGGL((paged_decode_mfma16_kernel<MKV_DTYPE_BF16, PAIR>), grid, block, 0, s, a);
      break;
    case MKV_DTYPE_F16:
      hipLaunchKernelGGL((paged_decode_mfma16_kernel<MKV_DTYPE_F16, PAIR>), grid, block, 0, s, a);
      break;
    default:
      hipLaunchKernelGGL(paged_decode_mfma32_kernel<PAIR>, grid, block, 0, s, a);
      break;
  }
  if (a.max_splits > 1) {
    const int64_t mitems = (int64_t)batch * a.num_heads;
    hipLaunchKernelGGL(paged_decode_merge_kernel, dim3((unsigned)((mitems + kDecWaves - 1) / kDecWaves)),
                       block, 0, s, a, (int)fp8);
  }
  return (int)hipGetLastError();
}

// Validate the arguments and fill the kernel arguments; returns the status
// and, on success, the call's kernel shape and format in ks / fmt.
int decode_args(void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride, int q_dtype,
                const void* k_cache, const void* v_cache, int kv_dtype, int64_t num_blocks,
                const float* k_scale, const float* v_scale, int kv_scale_mode,
                const int32_t* block_tables, int64_t bt_stride, int max_blocks, const void* context_lens,
                int context_lens_dtype, int batch, int num_heads, int num_kv_heads, int head_dim,
                int block_size, float sm_scale, int split_tokens, DecodeArgs& a, KernelShape& ks,
                int& fmt) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || max_blocks < 0 || num_blocks < 0)
    return MKV_ERR_BAD_SHAPE;
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens) return MKV_ERR_NULL_POINTER;
  const int shp = kernel_shape(num_heads, num_kv_heads, head_dim, ks);
  if (shp != MKV_OK) return shp;
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 4) return MKV_ERR_BAD_BLOCK_SIZE;
  if (q_dtype != MKV_DTYPE_F32 && q_dtype != MKV_DTYPE_BF16 && q_dtype != MKV_DTYPE_F16)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (kv_dtype != MKV_DTYPE_F32 && kv_dtype != MKV_DTYPE_BF16 && kv_dtype != MKV_DTYPE_F16 &&
      kv_dtype != MKV_DTYPE_FP8E4M3 && kv_dtype != MKV_DTYPE_I8)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  const bool quant = kv_dtype == MKV_DTYPE_FP8E4M3 || kv_dtype == MKV_DTYPE_I8;
  if (quant && kv_scale_mode != MKV_SCALE_PER_TENSOR && kv_scale_mode != MKV_SCALE_PER_TOKEN_HEAD)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  const bool per_token = quant && kv_scale_mode == MKV_SCALE_PER_TOKEN_HEAD;
  if (kv_dtype == MKV_DTYPE_I8 && !per_token) return MKV_ERR_UNSUPPORTED_DTYPE;
  if (quant && (!k_scale || !v_scale)) return MKV_ERR_NULL_POINTER;
  // per-token-head scale indices are 32-bit
  if (per_token && num_blocks * (int64_t)block_size * num_kv_heads >= (int64_t(1) << 31))
    return MKV_ERR_BAD_SHAPE;
  // kernel format: the dtype, or a per-token-head code
  fmt = per_token ? (kv_dtype == MKV_DTYPE_I8 ? kKvI8PerToken : kKvFp8PerToken) : kv_dtype;
  if (context_lens_dtype != MKV_INDEX_I32 && context_lens_dtype != MKV_INDEX_I64)
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (q_batch_stride < (int64_t)num_heads * head_dim || out_batch_stride < (int64_t)num_heads * head_dim ||
      bt_stride < max_blocks)
    return MKV_ERR_BAD_STRIDE;
  if (split_tokens != MKV_DECODE_WORKGROUP && split_tokens != MKV_DECODE_STREAM &&
      (split_tokens < 0 || split_tokens % 32 != 0))
    return MKV_ERR_BAD_SHAPE;
  const int qb = q_dtype == MKV_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u)
    return MKV_ERR_MISALIGNED;
  if ((q_batch_stride * qb) % 16 || (out_batch_stride * qb) % 16) return MKV_ERR_MISALIGNED;

  a = DecodeArgs{};
  a.out = out;
  a.out_stride = out_batch_stride;
  a.q = q;
  a.q_stride = q_batch_stride;
  a.q_dtype = q_dtype;
  a.k_cache = reinterpret_cast<const char*>(k_cache);
  a.v_cache = reinterpret_cast<const char*>(v_cache);
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
  a.batch = batch;
  a.num_heads = num_heads;
  a.num_kv_heads = ks.kv_heads;
  a.group = ks.group;
  a.scale_heads = num_kv_heads;
  a.pair = ks.pair ? 1 : 0;
  a.sm_scale = sm_scale;
  return MKV_OK;
}

int paged_decode_impl(void* out, int64_t out_batch_stride, const void* q, int64_t q_batch_stride,
                      int q_dtype, const void* k_cache, const void* v_cache, int kv_dtype,
                      int64_t num_blocks, const float* k_scale, const float* v_scale,
                      int kv_scale_mode, const int32_t* block_tables, int64_t bt_stride,
                      int max_blocks, const void* context_lens, int context_lens_dtype, int batch,
                      int num_heads, int num_kv_heads, int head_dim, int block_size,
                      float sm_scale, int split_tokens, void* workspace, size_t workspace_bytes,
                      void* stream, bool noalloc) {
  DecodeArgs a;
  KernelShape ks;
  int fmt = 0;
  const int st = decode_args(out, out_batch_stride, q, q_batch_stride, q_dtype, k_cache, v_cache, kv_dtype,
                             num_blocks, k_scale, v_scale, kv_scale_mode, block_tables, bt_stride, max_blocks,
                             context_lens, context_lens_dtype, batch, num_heads, num_kv_heads, head_dim,
                             block_size, sm_scale, split_tokens, a, ks, fmt);
  if (st != MKV_OK) return st;
  if (batch == 0) return MKV_OK;
  const int cus = device_cus();
  int route = choose_route(split_tokens, kv_dtype, batch, ks, max_blocks, block_size, cus,
                           fmt == kKvFp8PerToken || fmt == kKvI8PerToken);
  if (noalloc && route_ws_bytes(route, batch, num_heads, ks, max_blocks, block_size, split_tokens) >
                     workspace_bytes) {
    // The caller's scratch cannot hold this route's partials: the library's
    // choice falls back to the workgroup route (no workspace); an explicit
    // route is refused.
    if (split_tokens != 0) return MKV_ERR_SCRATCH_LIMIT;
    route = kRouteWorkgroup;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return ks.pair ? launch_route<true>(a, route, fmt, split_tokens, max_blocks, block_size, workspace,
                                      workspace_bytes, s)
                 : launch_route<false>(a, route, fmt, split_tokens, max_blocks, block_size, workspace,
                                       workspace_bytes, s);
}

}  // namespace

// Scratch of mkv_paged_decode_noalloc: one array per GPU, held from the
// library's first use on that GPU until the process ends.  It is sized for
// the stream-K partial slots of group sizes up to 8 on 256 CUs (2048 waves x
// 2 slots x 8 heads x 130 floats = 16.3 MiB, plus four ints per sequence:
// the tile prefix and the merge metadata) with room for moderate split-K
// requests (the workgroup route needs none); larger requests are
// refused.  Host code must not pass the array's name to a kernel: in host
// code it is a stand-in, not a device address.  The per-device address comes
// from hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kScratchBytes = MKV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array (resolved on the
// first call on that device).
int scratch_address(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MKV_ERR_BAD_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess) return (int)r;
    if (!p) return MKV_ERR_NULL_POINTER;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MKV_OK;
}

}  // namespace

extern "C" int mkv_paged_decode(void* out, int64_t out_batch_stride, const void* q,
                                int64_t q_batch_stride, int q_dtype, const void* k_cache,
                                const void* v_cache, int kv_dtype, int64_t num_blocks,
                                const float* k_scale, const float* v_scale, int kv_scale_mode,
                                const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                const void* context_lens, int context_lens_dtype, int batch,
                                int num_heads, int num_kv_heads, int head_dim, int block_size,
                                float sm_scale, int split_tokens, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return paged_decode_impl(out, out_batch_stride, q, q_batch_stride, q_dtype, k_cache, v_cache, kv_dtype,
                           num_blocks, k_scale, v_scale, kv_scale_mode, block_tables, bt_stride, max_blocks,
                           context_lens, context_lens_dtype, batch, num_heads, num_kv_heads, head_dim,
                           block_size, sm_scale, split_tokens, workspace, workspace_bytes, stream, false);
}

extern "C" int mkv_paged_decode_noalloc(void* out, int64_t out_batch_stride, const void* q,
                                        int64_t q_batch_stride, int q_dtype, const void* k_cache,
                                        const void* v_cache, int kv_dtype, int64_t num_blocks,
                                        const float* k_scale, const float* v_scale, int kv_scale_mode,
                                        const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                                        const void* context_lens, int context_lens_dtype, int batch,
                                        int num_heads, int num_kv_heads, int head_dim, int block_size,
                                        float sm_scale, int split_tokens, void* stream) {
  // An explicit route whose partials do not fit is refused on the host,
  // before the device is touched (the library's choice falls back instead).
  KernelShape ks;
  if (split_tokens != 0 && batch > 0 && max_blocks > 0 && block_size > 0 &&
      kernel_shape(num_heads, num_kv_heads, head_dim, ks) == MKV_OK) {
    const int route = choose_route(split_tokens, kv_dtype, batch, ks, max_blocks, block_size, device_cus());
    if (route_ws_bytes(route, batch, num_heads, ks, max_blocks, block_size, split_tokens) > kScratchBytes)
      return MKV_ERR_SCRATCH_LIMIT;
  }
  void* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st != MKV_OK) return st;
  return paged_decode_impl(out, out_batch_stride, q, q_batch_stride, q_dtype, k_cache, v_cache, kv_dtype,
                           num_blocks, k_scale, v_scale, kv_scale_mode, block_tables, bt_stride, max_blocks,
                           context_lens, context_lens_dtype, batch, num_heads, num_kv_heads, head_dim,
                           block_size, sm_scale, split_tokens, ws, kScratchBytes, stream, true);
}

extern "C" int mkv_qkv_norm_rope_append_decode(
    void* out, int64_t out_batch_stride, int out_dtype, const void* qkv, int64_t qkv_row_stride,
    int in_dtype, const void* q_norm_weight, const void* k_norm_weight, int norm_weight_dtype, float eps,
    const void* cos_sin_cache, int cos_sin_dtype, int64_t max_position, const int64_t* positions,
    void* k_cache, void* v_cache, int kv_dtype, int64_t num_blocks, float* k_scale, float* v_scale,
    int kv_scale_mode, const int64_t* slot_mapping, int flags, const int32_t* block_tables,
    int64_t bt_stride, int max_blocks, const void* context_lens, int context_lens_dtype, int batch,
    int num_heads, int num_kv_heads, int head_dim, int block_size, float sm_scale, void* stream) {
  DecodeArgs d;
  KernelShape ks;
  int fmt = 0;
  // the attention's arguments (q is produced in the kernel: qkv stands in
  // for its pointer in the checks)
  int st = decode_args(out, out_batch_stride, qkv, (int64_t)num_heads * head_dim, out_dtype, k_cache, v_cache,
                       kv_dtype, num_blocks, k_scale, v_scale, kv_scale_mode, block_tables, bt_stride, max_blocks,
                       context_lens, context_lens_dtype, batch, num_heads, num_kv_heads, head_dim, block_size,
                       sm_scale, MKV_DECODE_WORKGROUP, d, ks, fmt);
  if (st != MKV_OK) return st;
  if (head_dim != kHeadDim || ks.pair) return MKV_ERR_UNSUPPORTED_HEAD_DIM;
  // per-tensor FP8, fp16, or a bf16-MFMA format (bf16, per-token-head FP8 /
  // INT8) with a bf16 q: the workgroup route's kernel without the split q
  const bool bf16_mfma = fmt == MKV_DTYPE_BF16 || fmt == kKvFp8PerToken || fmt == kKvI8PerToken;
  if (fmt != MKV_DTYPE_FP8E4M3 && fmt != MKV_DTYPE_F16 && !(bf16_mfma && out_dtype == MKV_DTYPE_BF16))
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (d.group > kFusedMaxGroup) return MKV_ERR_UNSUPPORTED_GROUP;
  // the producer's arguments
  if (max_position <= 0) return MKV_ERR_BAD_SHAPE;
  if (!cos_sin_cache || !positions || !slot_mapping) return MKV_ERR_NULL_POINTER;
  auto is_float = [](int dt) { return dt == MKV_DTYPE_F32 || dt == MKV_DTYPE_BF16 || dt == MKV_DTYPE_F16; };
  if (!is_float(in_dtype) || !is_float(cos_sin_dtype) ||
      ((q_norm_weight || k_norm_weight) && !is_float(norm_weight_dtype)))
    return MKV_ERR_UNSUPPORTED_DTYPE;
  if (flags & ~MKV_APPEND_CALIBRATE_SENTINEL) return MKV_ERR_BAD_SHAPE;
  if (qkv_row_stride < (int64_t)(num_heads + 2 * num_kv_heads) * head_dim) return MKV_ERR_BAD_STRIDE;
  const int ib = in_dtype == MKV_DTYPE_F32 ? 4 : 2;
  const int cb = cos_sin_dtype == MKV_DTYPE_F32 ? 4 : 2;
  const int wb = norm_weight_dtype == MKV_DTYPE_F32 ? 4 : 2;
  auto misaligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; };
  if ((qkv_row_stride * ib) % 16 || misaligned(cos_sin_cache) || (head_dim * cb) % 16 ||
      (q_norm_weight && misaligned(q_norm_weight)) || (k_norm_weight && misaligned(k_norm_weight)) ||
      (head_dim / 2 * wb) % 16)
    return MKV_ERR_MISALIGNED;
  if (batch == 0) return MKV_OK;

  ProduceDecodeArgs f;
  f.d = d;
  f.d.q = nullptr;
  f.d.split_tokens = 0;
  f.d.max_splits = 0;
  ProducerArgs& p = f.p;
  p = ProducerArgs{};
  p.qkv = reinterpret_cast<const char*>(qkv);
  p.qkv_stride = qkv_row_stride;
  p.num_tokens = batch;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.q_w = q_norm_weight;
  p.k_w = k_norm_weight;
  p.w_dtype = norm_weight_dtype;
  p.eps = eps;
  p.cos_sin = cos_sin_cache;
  p.cs_dtype = cos_sin_dtype;
  p.max_position = max_position;
  p.positions = positions;
  p.out_dtype = out_dtype;
  p.k_cache = reinterpret_cast<char*>(k_cache);
  p.v_cache = reinterpret_cast<char*>(v_cache);
  p.cache_dtype = kv_dtype;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.calibrate = (flags & MKV_APPEND_CALIBRATE_SENTINEL) ? 1 : 0;
  p.slot_mapping = slot_mapping;
  p.num_slots = num_blocks * (int64_t)block_size;

  const int nw = wg_waves(batch, d.num_kv_heads, d.group, max_blocks, block_size, device_cus());
  const size_t row_bytes = (size_t)kHeadDim * (fmt == MKV_DTYPE_F16 || fmt == MKV_DTYPE_BF16 ? 2 : 1);
  const size_t lds = ((size_t)nw * d.group * (kHeadDim + 2) + (size_t)d.group * kHeadDim) * sizeof(float) +
                     2 * row_bytes;
  const dim3 grid((unsigned)((int64_t)batch * d.num_kv_heads)), block(nw * kWave);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define MKV_PD(IDT, KDT) hipLaunchKernelGGL((paged_decode_wg_produce_kernel<IDT, KDT>), grid, block, lds, s, f)
#define MKV_PD_KV(IDT)                                           \
  switch (fmt) {                                                 \
    case MKV_DTYPE_FP8E4M3: MKV_PD(IDT, MKV_DTYPE_FP8E4M3); break; \
    case kKvFp8PerToken: MKV_PD(IDT, kKvFp8PerToken); break;       \
    case kKvI8PerToken: MKV_PD(IDT, kKvI8PerToken); break;         \
    case MKV_DTYPE_BF16: MKV_PD(IDT, MKV_DTYPE_BF16); break;       \
    default: MKV_PD(IDT, MKV_DTYPE_F16); break;                    \
  }
  switch (in_dtype) {
    case MKV_DTYPE_BF16: MKV_PD_KV(MKV_DTYPE_BF16); break;
    case MKV_DTYPE_F16: MKV_PD_KV(MKV_DTYPE_F16); break;
    default: MKV_PD_KV(MKV_DTYPE_F32); break;
  }
#undef MKV_PD_KV
#undef MKV_PD
  return (int)hipGetLastError();
}
