"""CPU tests of the host side: the C-ABI library, the Python wrappers'
argument handling, the per-step metadata helpers and the workloads.  No
kernel is launched here (there is no GPU in this environment)."""
from __future__ import annotations

import ctypes
import re

import pytest
import torch

from conftest import REPO
from mkv import _lib
from mkv import attention as A
from mkv import context as C
from mkv import workloads as W


def _declared_functions() -> set[str]:
    text = (REPO / "include" / "mkv.h").read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(mkv_\w+)\s*\(", text, flags=re.M))


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    for n in ("mkv_kv_append", "mkv_kv_append_per_token_head", "mkv_fp8_calibrate_per_tensor",
              "mkv_paged_decode", "mkv_decode_metadata", "mkv_qkv_norm_rope_append",
              "mkv_paged_prefill", "mkv_flash_prefill", "mkv_gather_kv", "mkv_abi_version",
              "mkv_status_string"):
        assert n in names


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.mkv_abi_version() == _lib.ABI_VERSION


def test_status_strings():
    lib = _lib.load()
    for code in range(0, -11, -1):
        s = lib.mkv_status_string(code).decode()
        assert s and s != "unknown mkv status"
    assert lib.mkv_status_string(-1234).decode() == "unknown mkv status"


def test_fused_decode_step_refuses_what_it_does_not_cover():
    """mkv_qkv_norm_rope_append_decode checks its arguments on the host,
    before any launch: an fp32 cache, a bf16 or per-token-head cache under
    a q other than bf16 (whose decode splits q in two bf16 parts), head_dim 64
    and 16 query heads per KV head are refused (the caller runs the producer
    and the decode instead), and so are a missing slot mapping and a short
    qkv row."""
    lib = _lib.load()
    P = 1 << 12  # an aligned stand-in address: nothing is dereferenced

    def call(kv_dtype=_lib.DTYPE_FP8E4M3, Hq=16, Hkv=8, D=128, slots=P, qkv_stride=None,
             out_dtype=_lib.DTYPE_BF16, scale_mode=_lib.SCALE_PER_TENSOR):
        width = (Hq + 2 * Hkv) * D
        return lib.mkv_qkv_norm_rope_append_decode(
            P, Hq * D, out_dtype, P, width if qkv_stride is None else qkv_stride, _lib.DTYPE_BF16,
            P, P, _lib.DTYPE_BF16, 1e-6, P, _lib.DTYPE_BF16, 4096, P, P, P, kv_dtype, 64, P, P,
            scale_mode, slots, 0, P, 4, 4, P, _lib.INDEX_I64, 60, Hq, Hkv, D, 256, 0.088,
            None)

    assert call(kv_dtype=_lib.DTYPE_F32) == -3
    assert call(kv_dtype=_lib.DTYPE_BF16, out_dtype=_lib.DTYPE_F32) == -3
    assert call(scale_mode=_lib.SCALE_PER_TOKEN_HEAD, out_dtype=_lib.DTYPE_F32) == -3
    assert call(kv_dtype=_lib.DTYPE_I8, scale_mode=_lib.SCALE_PER_TOKEN_HEAD, out_dtype=_lib.DTYPE_F16) == -3
    assert call(Hq=16, Hkv=8, D=64) == -4
    assert call(Hq=128, Hkv=8) == -5
    assert call(slots=None) == -1
    assert call(qkv_stride=100) == -9


def test_noalloc_decode_refuses_requests_beyond_its_scratch():
    """The allocation-free decode checks its scratch limit on the host,
    before it touches the device."""
    lib = _lib.load()
    args = [None, 32 * 128, None, 32 * 128, _lib.DTYPE_BF16, None, None, _lib.DTYPE_F32, 4096,
            None, None, 0, None, 32, 32, None, _lib.INDEX_I64, 1024, 32, 8, 128, 256, 0.088, 32,
            None]
    # split-K partials of 1024 x 32 heads x 256 splits: 4.4 GB > 32 MiB
    assert lib.mkv_paged_decode_noalloc(*args) == -10
    assert lib.mkv_paged_decode_workspace_size(1024, 32, 8, 32, 256, 128, _lib.DTYPE_F32, 32) \
        > _lib.NOALLOC_SCRATCH_BYTES
    assert "scratch" in lib.mkv_status_string(-10).decode()


def test_argument_validation_without_launch():
    """Bad arguments are rejected before any device work is enqueued."""
    lib = _lib.load()
    nul = None
    # null pointers
    assert lib.mkv_kv_append(nul, 1024, nul, 1024, nul, nul, nul, 4, 8, 128, 16, 4, 1, 3,
                             nul, nul, 0, nul) == -1
    # unsupported head_dim / group / block size in decode
    p = ctypes.c_void_p(16)
    base = [p, 4096, p, 4096, 1, p, p, 1, 10, nul, nul, 0, p, 4, 4, p, 1, 2]
    assert lib.mkv_paged_decode(*base, 32, 8, 96, 256, 0.1, 0, nul, 0, nul) == -4
    # head_dim 64 pairs KV heads: an odd KV-head count, or more than 8 query
    # heads per KV head, is rejected
    assert lib.mkv_paged_decode(*base, 21, 7, 64, 256, 0.1, 0, nul, 0, nul) == -4
    assert lib.mkv_paged_decode(*base, 32, 2, 64, 256, 0.1, 0, nul, 0, nul) == -5
    assert lib.mkv_paged_decode(*base, 32, 6, 128, 256, 0.1, 0, nul, 0, nul) == -5
    assert lib.mkv_paged_decode(*base, 32, 8, 128, 100, 0.1, 0, nul, 0, nul) == -6
    assert lib.mkv_paged_decode(*base, 32, 8, 128, 8, 0.1, 0, nul, 0, nul) == -6
    # workspace too small for a split-K launch
    assert lib.mkv_paged_decode(*base, 32, 8, 128, 256, 0.1, 32, p, 16, nul) == -7
    # zero tokens / batch is a no-op that succeeds
    assert lib.mkv_kv_append(nul, 1024, nul, 1024, nul, nul, nul, 0, 8, 128, 16, 4, 1, 3,
                             nul, nul, 0, nul) == 0
    # unknown append flags are rejected
    assert lib.mkv_kv_append(p, 1024, p, 1024, p, p, p, 4, 8, 128, 16, 4, 1, 3, p, p, 6,
                             nul) == -2
    # quantised caches: INT8 needs per-token-head scales, scales must be given,
    # and an unknown scale mode is rejected
    q8 = [p, 4096, p, 4096, 1, p, p]
    tail = [p, 4, 4, p, 1, 2, 32, 8, 128, 256, 0.1, 0, p, 1 << 20, nul]
    assert lib.mkv_paged_decode(*q8, 4, 10, p, p, 0, *tail) == -3
    assert lib.mkv_paged_decode(*q8, 4, 10, nul, p, 1, *tail) == -1
    assert lib.mkv_paged_decode(*q8, 3, 10, p, p, 7, *tail) == -3
    # per-token-head append: head_dim must be a power of two in 16..1024,
    # the cache FP8 or INT8
    assert lib.mkv_kv_append_per_token_head(p, 1024, p, 1024, p, p, p, p, p, 4, 8, 96, 16, 4,
                                            1, 3, nul) == -4
    assert lib.mkv_kv_append_per_token_head(p, 1024, p, 1024, p, p, p, p, p, 4, 8, 128, 16, 4,
                                            1, 1, nul) == -3
    assert lib.mkv_kv_append_per_token_head(p, 1024, p, 1024, p, p, nul, p, p, 4, 8, 128, 16, 4,
                                            1, 4, nul) == -1
    # decode metadata: nothing to do for zero rows; bad block size / pointers
    assert lib.mkv_decode_metadata(nul, nul, nul, nul, 8, 8, 10, 16, 0, 1, nul) == 0
    assert lib.mkv_decode_metadata(p, p, p, p, 8, 8, 10, 24, 4, 1, nul) == -6
    assert lib.mkv_decode_metadata(p, nul, p, p, 8, 8, 10, 16, 4, 1, nul) == -1
    assert lib.mkv_decode_metadata(p, p, p, p, 4, 8, 10, 16, 4, 1, nul) == -9
    # fused producer: head_dim must be a power of two >= 32; INT8 needs
    # per-token-head scales; unknown flags are rejected
    prod = [p, 4096, 1, 4, 16, 8, 128, nul, nul, 1, 1e-5, p, 0, 64, p, p, nul, 1, p, p, 3, 0, p, p,
            p, 16, 8, 0, nul]
    bad = list(prod)
    bad[6] = 96
    assert lib.mkv_qkv_norm_rope_append(*bad) == -4
    bad = list(prod)
    bad[20], bad[21] = 4, 0
    assert lib.mkv_qkv_norm_rope_append(*bad) == -3
    bad = list(prod)
    bad[27] = 4
    assert lib.mkv_qkv_norm_rope_append(*bad) == -2
    # prefill scale modes: FP8 takes per-tensor or per-token-head scales,
    # INT8 only per-token-head ones, and a quantised cache needs both scales
    pre = [p, p, 1, p, p, 3, 10, p, p, 7, p, 4, 4, p, 1, p, p, 1, 4, 32, 8, 128, 256, 0.1,
           p, 1 << 20, nul]
    assert lib.mkv_paged_prefill(*pre) == -3  # unknown scale mode
    pre[5], pre[9] = 4, 0  # INT8 with a per-tensor scale
    assert lib.mkv_paged_prefill(*pre) == -3
    pre[9], pre[7] = 1, nul  # INT8 per token and head without its K scales
    assert lib.mkv_paged_prefill(*pre) == -1
    pre[5] = 3  # FP8 per token and head without its K scales
    assert lib.mkv_paged_prefill(*pre) == -1


def test_decode_workspace_and_split_queries():
    lib = _lib.load()
    F32, BF16, FP8 = _lib.DTYPE_F32, _lib.DTYPE_BF16, _lib.DTYPE_FP8E4M3
    st = lib.mkv_paged_decode_split_tokens(256, 8, 32, 256, 0)
    assert st % 32 == 0 and 64 <= st <= 512
    # an fp32 cache always takes split-K: its partials
    n = lib.mkv_paged_decode_workspace_size(256, 32, 8, 32, 256, 128, F32, 0)
    splits = (32 * 256 + st - 1) // st
    assert n == 256 * 32 * splits * 130 * 4
    # explicit split sizes select the split-K path only
    n512 = lib.mkv_paged_decode_workspace_size(256, 32, 8, 32, 256, 128, FP8, 512)
    assert n512 == 256 * 32 * 16 * 130 * 4
    # one split covers the table: no workspace on the split-K path
    assert lib.mkv_paged_decode_workspace_size(4, 16, 8, 1, 256, 128, FP8, 512) == 0
    st4 = lib.mkv_paged_decode_split_tokens(4, 8, 1, 256, 0)
    splits4 = (256 + st4 - 1) // st4
    assert lib.mkv_paged_decode_workspace_size(4, 16, 8, 1, 256, 128, F32, 0) == (
        4 * 16 * splits4 * 130 * 4 if splits4 > 1 else 0)
    # the default stream-K route needs its partial slots for the persistent
    # grid and the per-sequence metadata only, not the split-K partials: without a GPU
    # the CU count query falls back to 512 CUs, i.e. 4096 waves
    nsk = lib.mkv_paged_decode_workspace_size(256, 32, 8, 32, 256, 128, FP8, 0)
    assert lib.mkv_paged_decode_workspace_size(256, 32, 8, 32, 256, 128, BF16, 0) == nsk
    # (per sequence: the tile prefix and three merge-metadata words)
    assert nsk % (2 * 4 * 130 * 4) == (4 * 256 + 2) * 4
    waves = (nsk - (4 * 256 + 2) * 4) // (2 * 4 * 130 * 4)
    assert waves in (4096, 2048) and nsk < n
    # (a 1-block table: 32 tokens a wave take the workgroup route, no
    # workspace; 16 blocks take stream-K)
    assert lib.mkv_paged_decode_workspace_size(4, 16, 8, 1, 256, 128, BF16, 0) == 0
    assert lib.mkv_paged_decode_workspace_size(4, 16, 8, 16, 256, 128, FP8, 0) > 0
    # FP8 at 256 tokens a wave: per-tensor scales take the workgroup route at
    # this fill, per-token-head scales stream-K; the query, which has no
    # scale mode, sizes for the larger
    assert lib.mkv_paged_decode_workspace_size(8, 32, 8, 8, 256, 128, FP8, 0) > 0
    # small batches split finer
    assert lib.mkv_paged_decode_split_tokens(4, 8, 8, 256, 0) < st or st == 64


def test_decode_route_choice():
    """The library's schedule for split_tokens 0 (mkv_paged_decode_route on
    a 256-CU device), for the decode workloads that are measured, and the
    explicit overrides."""
    lib = _lib.load()
    F32, FP8, BF16 = _lib.DTYPE_F32, _lib.DTYPE_FP8E4M3, _lib.DTYPE_BF16
    SK, SP, WG = _lib.ROUTE_STREAM, _lib.ROUTE_SPLIT, _lib.ROUTE_WORKGROUP

    def route(B, Hq, Hkv, mb, bs, D, dt, st=0):
        return lib.mkv_paged_decode_route(B, Hq, Hkv, mb, bs, D, dt, st, 256)

    # batch 256, 32 / 8 heads, contexts up to 8192 in 32-block tables: stream-K
    assert route(256, 32, 8, 32, 256, 128, FP8) == SK
    assert route(256, 32, 8, 32, 256, 128, BF16) == SK
    # batch 32 over the appended pool, contexts up to 4096 (16-block tables):
    # a workgroup wave would take up to 512 tokens -> stream-K
    assert route(32, 32, 8, 16, 256, 128, FP8) == SK
    # the end-to-end engine's decode rows: 60 (bucket 64) sequences of at most
    # 768 tokens, 16 / 8 heads, tables padded to 4 blocks -> workgroup
    assert route(60, 16, 8, 4, 256, 128, FP8) == WG
    assert route(64, 16, 8, 4, 256, 128, FP8) == WG
    # the same rows in tables padded to max_model_len 4096 (16 blocks): stream-K
    assert route(60, 16, 8, 16, 256, 128, FP8) == SK
    # fp32 batch 4: too few workgroups -> split-K; batch 60 in 16-block tables:
    # workgroup (up to 512 tokens per wave for fp32)
    assert route(4, 16, 8, 8, 256, 128, F32) == SP
    assert route(60, 16, 8, 4, 256, 128, F32) == WG
    # small batches: at most 128 tokens a wave (4-block tables, 8 waves) take
    # the workgroup route whatever the fill; 256 tokens a wave only with the
    # fill (FP8 2 x CUs, 16-bit 6 x CUs, INT8 per-token-head never)
    I8 = _lib.DTYPE_I8
    for B in (1, 4):
        for dt in (FP8, BF16, I8):
            assert route(B, 16, 8, 4, 256, 128, dt) == WG
        assert route(B, 32, 8, 8, 256, 128, FP8) == SK
        assert route(B, 32, 8, 8, 256, 128, BF16) == SK
    assert route(8, 32, 8, 8, 256, 128, FP8) == WG
    assert route(8, 32, 8, 8, 256, 128, BF16) == SK
    assert route(32, 32, 8, 8, 256, 128, BF16) == WG
    assert route(60, 16, 8, 4, 256, 128, I8) == SK
    # head_dim 64 pairs KV heads: Llama-3.2-1B decode, batch 48, 12-block tables
    assert route(48, 32, 8, 12, 256, 64, FP8) == SK
    assert route(64, 32, 8, 2, 256, 64, BF16) == WG
    # explicit schedules
    assert route(60, 16, 8, 4, 256, 128, FP8, _lib.DECODE_STREAM) == SK
    assert route(60, 16, 8, 4, 256, 128, F32, _lib.DECODE_STREAM) == SP
    assert route(256, 32, 8, 32, 256, 128, FP8, _lib.DECODE_WORKGROUP) == WG
    assert route(256, 32, 8, 32, 256, 128, FP8, 256) == SP
    # unsupported shapes report their status
    assert route(4, 16, 8, 8, 256, 96, FP8) == -4
    assert route(4, 21, 7, 8, 256, 64, FP8) == -4


def test_wrappers_reject_cpu_tensors_and_unimplemented_modes():
    k = torch.zeros(2, 8, 128)
    kc = torch.zeros(1, 16, 8, 128)
    slots = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="no CPU fallback"):
        A.store_kvcache(k, k, kc, kc, slots, 16)
    with pytest.raises(TypeError, match="fp8 cache expected"):
        A.store_kvcache_fp8(k, k, kc, kc, None, None, slots, 16, "fp8_per_token_head")
    with pytest.raises(TypeError, match="int8 cache"):
        A.paged_attention_decode_quantized(k, kc, kc, None, None, None, None, 0.1, 8, 8, 128, 16,
                                           "int8_per_token_head")
    with pytest.raises(ValueError, match="unknown"):
        A.paged_attention_decode_quantized(k, kc, kc, None, None, None, None, 0.1, 8, 8, 128, 16,
                                           "fp4")
    bt, cl, cu = torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int64), torch.tensor([0, 2])
    with pytest.raises(ValueError, match="no CPU fallback"):
        A.paged_attention_prefill_triton(k, kc, kc, bt, cl, cu, torch.zeros(2, dtype=torch.int64), 0.1,
                                         8, 8, 128, 16, kv_cache_dtype="fp8_per_token_head")
    with pytest.raises(AssertionError):
        A.store_kvcache(k, k, kc, torch.zeros(2, 16, 8, 128), slots, 16)
    with pytest.raises(AssertionError):
        A.store_kvcache(k, k, kc, kc, torch.zeros(3, dtype=torch.int64), 16)
    layer = A.Attention(8, 128, num_kv_heads=8)
    layer.kv_cache_dtype = "kivi_2bit"
    with pytest.raises(NotImplementedError):
        layer(torch.zeros(1, 8, 128), k[:1], k[:1])


def test_mixed_split_metadata_matches_reference_rules():
    cu = [0, 4, 5, 6, 9]
    qlens = [4, 1, 1, 3]
    dec = [False, True, True, False]
    s = C.split_mixed_decode_prefill_metadata(cu, qlens, dec)
    assert s.decode_token_indices == [4, 5]
    assert s.decode_seq_indices == [1, 2]
    assert s.prefill_token_indices == [0, 1, 2, 3, 6, 7, 8]
    assert s.prefill_seq_indices == [0, 3]
    assert s.prefill_cu_seqlens_q == [0, 4, 7]
    t = C.split_mixed_decode_prefill_metadata(torch.tensor(cu), torch.tensor(qlens), torch.tensor(dec))
    assert t == s


def test_context_round_trip():
    C.set_context(True, cu_seqlens_q=torch.tensor([0, 3]), max_seqlen_q=3, is_full_prefill=True)
    ctx = C.get_context()
    assert ctx.is_prefill and ctx.max_seqlen_q == 3 and ctx.is_full_prefill
    C.reset_context()
    assert C.get_context() == C.Context()


def test_workloads_are_seeded_and_consistent():
    a, b = W.decode_small(1), W.decode_small(1)
    assert torch.equal(a["q"], b["q"]) and torch.equal(a["block_tables"], b["block_tables"])
    bt, ctx = a["block_tables"], a["context_lens"]
    used = bt[bt >= 0]
    assert used.unique().numel() == used.numel()  # fragmented but disjoint
    for i in range(bt.shape[0]):
        nb = (int(ctx[i]) + 255) // 256
        assert (bt[i, :nb] >= 0).all() and (bt[i, nb:] == -1).all()
    m = W.decode_b256_metadata(3)
    L = m["context_lens"]
    assert L.min() >= 512 and L.max() < 8192 and 2000 < float(L.float().mean()) < 3600
    ap = W.append_fp8(2)
    s = ap["slot_mapping"]
    v = s[s >= 0]
    assert v.unique().numel() == v.numel() and 0.03 < float((s < 0).float().mean()) < 0.07
    pm = W.prefill_mixed(4)
    assert int(pm["cu_seqlens_q"][-1]) == 8 * 512 + 120 == pm["positions"].numel()


def test_algorithmic_bytes():
    ctx = torch.tensor([512, 1000])
    n = W.alg_bytes_decode(ctx, 256, 32, 8, kv_bytes=1)
    assert n == 1512 * 8 * 128 * 2 + 2 * 32 * 128 * 4 + (2 + 4) * 4 + 2 * 8


def test_context_provider_hook():
    """Attention can read an engine-owned context object (same field names)."""
    class EngineContext:
        is_prefill = True
    C.use_context_provider(lambda: EngineContext)
    try:
        assert C.current_context() is EngineContext
    finally:
        C.use_context_provider(None)
    assert C.current_context() is C.get_context()


def test_key_and_value_reach_the_abi_in_one_dtype(monkeypatch):
    """The C ABI reads key and value with one element dtype.  A rotated k
    promoted to fp32 (an fp32 cos/sin table) next to a bf16 v once reached it
    with the key's dtype, so the kernel read the v buffer at twice its size.
    Every wrapper must now pass rows of one dtype (widened to fp32, exact),
    cast both to the cache dtype in copy mode, and calibrate per tensor."""
    seen, calls = [], []
    real_rows = A._token_rows

    def rows(x):
        out = real_rows(x)
        seen.append(out)
        return out

    monkeypatch.setattr(A, "_token_rows", rows)
    monkeypatch.setattr(A, "_require_gpu", lambda *t: torch.device("cpu"))
    monkeypatch.setattr(A, "_stream", lambda dev: 0)
    monkeypatch.setattr(A, "_workspace", lambda dev, name, n, zeroed=False: torch.zeros(max(n, 256), dtype=torch.uint8))
    monkeypatch.setattr(A._lib, "call", lambda name, *args: calls.append((name, args)))
    monkeypatch.setattr(A._lib, "query", lambda name, *args: 16)
    key = torch.randn(4, 8, 128)  # fp32
    value = torch.randn(4, 8, 128).to(torch.bfloat16)
    slots = torch.arange(4)

    def last_pair():
        k, v = seen[-2], seen[-1]
        assert k.dtype == v.dtype and k.shape == v.shape
        return k, v

    # FP8 per tensor: widened to fp32, in-kernel calibration off for the pair
    kc = torch.zeros(2, 16, 8, 128, dtype=torch.float8_e4m3fn)
    A._append(key, value, kc, kc.clone(), slots, torch.ones(1), torch.ones(1), calibrate_sentinel=True)
    k, v = last_pair()
    assert k.dtype == torch.float32 and torch.equal(v, value.float())
    name, args = calls[-1]
    assert name == "mkv_kv_append" and args[12] == _lib.DTYPE_F32 and args[16] == 0
    # copy mode: each cast to the cache dtype
    kb = torch.zeros(2, 16, 8, 128, dtype=torch.bfloat16)
    A._append(key, value, kb, kb.clone(), slots)
    k, v = last_pair()
    assert k.dtype == torch.bfloat16 and calls[-1][1][12] == _lib.DTYPE_BF16
    # per-token-head
    kq = torch.zeros(2, 16, 8, 128, dtype=torch.int8)
    A._append_per_token_head(key, value, kq, kq.clone(), torch.ones(2, 16, 8), torch.ones(2, 16, 8), slots)
    k, v = last_pair()
    assert k.dtype == torch.float32 and calls[-1][1][14] == _lib.DTYPE_F32
    # calibration: one launch per tensor, each in its own dtype
    calls.clear()
    A.calibrate_fp8_per_tensor(key, value, torch.ones(1), torch.ones(1))
    assert [c[0] for c in calls] == ["mkv_fp8_calibrate_per_tensor"] * 2
    assert calls[0][1][6] == _lib.DTYPE_F32 and calls[1][1][6] == _lib.DTYPE_BF16
    # mismatched shapes or cache dtypes are refused before any launch
    with pytest.raises(ValueError):
        A._append(key, value[:3], kc, kc.clone(), slots, torch.ones(1), torch.ones(1))
    with pytest.raises(TypeError):
        A._append(key, value, kc, kb, slots, torch.ones(1), torch.ones(1))


def test_bench_extra_selection():
    """bench.py's --extra picks secondary measurements by name (for profiling
    one workload at a time) and refuses unknown names before any GPU work."""
    import sys
    sys.path.insert(0, str(REPO))
    import bench
    assert bench.parse_args([]).extra_set == set(bench.EXTRAS)
    assert bench.parse_args(["--extra", "prefill, mixed"]).extra_set == {"prefill", "mixed"}
    assert bench.parse_args(["--no-extra", "--extra", "prefill"]).extra_set == set()
    with pytest.raises(SystemExit):
        bench.parse_args(["--extra", "prefil"])


def test_assert_close_out_rejects_nan_differences():
    """The GPU tests' tolerance check fails a NaN on one side only (a bare
    `err > tol` is False for NaN and would pass it) and accepts NaN on both."""
    from conftest import assert_close_out
    want = torch.tensor([1.0, float("nan"), 2.0])
    assert_close_out(torch.tensor([1.0, float("nan"), 2.0]), want, torch.float32, 1e-3)
    for got in (torch.tensor([float("nan"), float("nan"), 2.0]), torch.tensor([1.0, 1.0, 2.0]),
                torch.tensor([1.0, float("nan"), float("inf")])):
        with pytest.raises(AssertionError):
            assert_close_out(got, want, torch.float32, 1e-3)


def test_stream_read_probe_checks_arguments_on_the_host():
    """The read probe (a measurement helper) refuses bad sizes, null and
    misaligned buffers before it launches anything."""
    lib = _lib.load()
    assert lib.mkv_stream_read_probe_sink_words(2048) == 2048 * 4
    assert lib.mkv_stream_read_probe_sink_words(0) == 0
    assert lib.mkv_stream_read_probe(16, 100, 16, 64, None) == -2      # bytes not a multiple of 16
    assert lib.mkv_stream_read_probe(16, 4096, 16, 0, None) == -2      # empty grid
    assert lib.mkv_stream_read_probe(16, 4096, 16, (1 << 20) + 1, None) == -2  # grid too large (above 2^20)
    assert lib.mkv_stream_read_probe(None, 4096, 16, 64, None) == -1
    assert lib.mkv_stream_read_probe(24, 4096, 16, 64, None) == -8     # misaligned buffer


def test_graph_capture_runs_the_collector_first_and_holds_it_off(monkeypatch):
    """A cycle collected inside a capture frees what it owns there (a dead
    engine's graphs and their pool), which aborts a capturing process: the
    capture helper collects first and keeps the collector off until the
    capture ends, an error in it included, and restores its state."""
    import contextlib
    import gc

    from mkv import decode_state as DS

    seen = []

    @contextlib.contextmanager
    def fake_graph(graph, pool=None):
        seen.append(("enter", gc.isenabled(), pool))
        yield
        seen.append(("exit", gc.isenabled()))

    class Cycle:
        def __init__(self):
            self.me = self

        def __del__(self):
            seen.append("collected")

    monkeypatch.setattr(DS.torch.cuda, "graph", fake_graph)
    assert gc.isenabled()
    Cycle()  # garbage only a collection frees
    with DS.graph_capture(object(), pool="p"):
        assert not gc.isenabled()
    assert seen == ["collected", ("enter", False, "p"), ("exit", False)]
    assert gc.isenabled()
    with pytest.raises(RuntimeError):
        with DS.graph_capture(object()):
            raise RuntimeError("step failed under capture")
    assert gc.isenabled()
    gc.disable()
    try:
        with DS.graph_capture(object()):
            pass
        assert not gc.isenabled()  # a caller's disabled collector stays disabled
    finally:
        gc.enable()
