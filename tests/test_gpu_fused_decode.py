"""GPU parity of the fused decode step (``mkv_qkv_norm_rope_append_decode``):
one layer's producer step for each sequence's new token (q/k RMSNorm,
rotary embedding, FP8, per-token-head or 16-bit append; reference qwen3.py:73-118,
attention.py:1654-1691) and the decode attention over the cache that holds
it (attention.py:1213-1268), in one launch.

* Against the two calls it replaces (mkv_qkv_norm_rope_append, then
  mkv_paged_decode on the workgroup route): the output, the appended cache
  bytes and the scales are bit-identical, over group sizes 1-8, block
  sizes 16 and 256, contexts 0-800 (the new token in a wave's first,
  second or a later tile), rows without a slot, every input dtype and the
  1.0-sentinel calibration; bf16, fp16 and per-token-head FP8 / INT8
  caches (loaded after the append has landed) over groups 1-8.
* Against the oracle (qkv_norm_rope_ref, then paged_decode_ref on the
  dequantised cache): within the FP8 bound, 2e-2 abs.
"""
from __future__ import annotations

import pytest
import torch

from conftest import announce, assert_close_out
from mkv import _lib
from mkv import attention as A
from mkv import producer as P
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu
D = 128
CTX_EDGES = [0, 1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513]


def _case(dev, seed, B, Hq, Hkv, bs, in_dtype, ctx=None, no_slot=(), scale_val=None,
          cache_dtype=torch.float8_e4m3fn, per_token=False):
    g = torch.Generator().manual_seed(seed)
    if ctx is None:
        ctx = torch.tensor((CTX_EDGES * ((B + len(CTX_EDGES) - 1) // len(CTX_EDGES)))[:B])
        ctx[B // 2:] = torch.randint(300, 801, (B - B // 2,), generator=g)
    ctx = torch.as_tensor(ctx, dtype=torch.int64)
    N = int(sum((int(c) + bs - 1) // bs for c in ctx)) + 8
    bt = W.fragmented_block_tables(ctx, bs, N, g)
    slots = torch.full((B,), -1, dtype=torch.int64)
    for b in range(B):
        L = int(ctx[b])
        if L > 0 and b not in no_slot:
            slots[b] = int(bt[b, (L - 1) // bs]) * bs + (L - 1) % bs
    pos = (ctx - 1).clamp(min=0)
    width = (Hq + 2 * Hkv) * D
    qkv = (torch.randn(B, width, generator=g) * 2).to(in_dtype)
    cs = R.rope_cos_sin_cache(1000000.0, D, 4096).to(in_dtype)
    qw = (torch.rand(D, generator=g) + 0.5).to(in_dtype)
    kw = (torch.rand(D, generator=g) + 0.5).to(in_dtype)
    kc = torch.empty(N, bs, Hkv, D, dtype=cache_dtype, device=dev)
    vc = torch.empty_like(kc)
    sk = 0.02 if scale_val is None else scale_val
    sv = 0.03 if scale_val is None else scale_val
    fp8 = cache_dtype == torch.float8_e4m3fn
    if per_token:
        kv = "int8_per_token_head" if cache_dtype == torch.int8 else "fp8_per_token_head"
        ks = torch.empty(N, bs, Hkv, dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        W.fill_pools_per_token_head_on_device(kc, vc, ks, vs, seed + 1, kv)
    else:
        kv = "fp8_per_tensor" if fp8 else "auto"
        W.fill_pool_on_device(kc, seed + 1, sk)
        W.fill_pool_on_device(vc, seed + 2, sv)
        ks = torch.full((1,), sk, device=dev) if fp8 else None
        vs = torch.full((1,), sv, device=dev) if fp8 else None
    return dict(qkv=qkv.to(dev), pos=pos.to(dev), cs=cs.to(dev), qw=qw.to(dev), kw=kw.to(dev), kc=kc,
                vc=vc, ks=ks, vs=vs, slots=slots.to(dev), bt=bt.to(dev), ctx=ctx.to(dev), B=B, Hq=Hq,
                Hkv=Hkv, bs=bs, scale=D ** -0.5, kv=kv)


def _calibrated(t):
    if t is not None:
        t = t.clone()
        t._mkv_calibrated = True
    return t


def _two_calls(c):
    kc, vc = c["kc"].clone(), c["vc"].clone()
    ks, vs = _calibrated(c["ks"]), _calibrated(c["vs"])
    q, _, _ = P.qkv_norm_rope_append(
        c["qkv"], c["pos"], c["Hq"], c["Hkv"], D, c["cs"], kc, vc, c["slots"], c["bs"],
        q_norm_weight=c["qw"], k_norm_weight=c["kw"], kv_cache_dtype=c["kv"], k_scale=ks,
        v_scale=vs)
    out = A._decode(q, kc, vc, c["bt"], c["ctx"], c["scale"], c["Hq"], c["Hkv"], D, ks, vs,
                    split_tokens=A.DECODE_WORKGROUP, per_token_head=c["kv"] in A.PER_TOKEN_HEAD_MODES)
    return out, kc, vc, ks, vs, q


def _fused(c):
    kc, vc = c["kc"].clone(), c["vc"].clone()
    ks, vs = _calibrated(c["ks"]), _calibrated(c["vs"])
    calls = []
    orig = _lib.call

    def spy(name, *args):
        calls.append(name)
        return orig(name, *args)

    _lib.call = spy
    try:
        out = P.qkv_norm_rope_append_decode(
            c["qkv"], c["pos"], c["Hq"], c["Hkv"], D, c["cs"], kc, vc, c["slots"], c["bs"], c["bt"],
            c["ctx"], c["scale"], q_norm_weight=c["qw"], k_norm_weight=c["kw"],
            kv_cache_dtype=c["kv"], k_scale=ks, v_scale=vs, split_tokens=A.DECODE_WORKGROUP)
    finally:
        _lib.call = orig
    assert calls == ["mkv_qkv_norm_rope_append_decode"], calls
    return out, kc, vc, ks, vs


def _assert_same(f, u):
    out, kc, vc, ks, vs = f
    out_u, kc_u, vc_u, ks_u, vs_u = u[:5]
    assert torch.equal(kc.view(torch.uint8), kc_u.view(torch.uint8)), "K cache bytes differ"
    assert torch.equal(vc.view(torch.uint8), vc_u.view(torch.uint8)), "V cache bytes differ"
    if ks is not None:
        assert torch.equal(ks, ks_u) and torch.equal(vs, vs_u), "scales differ"
    diff = (out.float() != out_u.float()) & ~(torch.isnan(out.float()) & torch.isnan(out_u.float()))
    assert not bool(diff.any()), (f"{int(diff.sum())} outputs differ, max "
                                  f"{float((out.float() - out_u.float()).abs().max()):.3e}")


@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 8), (8, 8), (48, 8), (56, 8), (64, 8), (12, 2), (24, 3)])
@pytest.mark.parametrize("bs", [16, 256])
def test_fused_decode_step_equals_the_two_calls(dev, Hq, Hkv, bs):
    announce(f"fused decode step {Hq}/{Hkv} block {bs}")
    c = _case(dev, Hq * 7 + bs, 40, Hq, Hkv, bs, torch.bfloat16, no_slot=(5, 21))
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 8), (8, 8), (64, 8), (24, 3), (12, 4), (40, 8), (48, 8),
                                    (56, 8)])
@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bs", [16, 256])
def test_fused_decode_step_16bit_caches(dev, Hq, Hkv, cache_dtype, bs):
    """bf16 (with a bf16 q) and fp16 caches: the rows are appended as the
    producer's cast, and the attention reads every tile after the append."""
    announce(f"fused decode step {cache_dtype} cache {Hq}/{Hkv} block {bs}")
    c = _case(dev, Hq * 5 + bs + 1, 40, Hq, Hkv, bs, torch.bfloat16, no_slot=(4, 30),
              cache_dtype=cache_dtype)
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_fused_decode_step_other_block_sizes(dev, bs, cache_dtype):
    """Block sizes between the two above: the row patch's (1-byte) and the
    tiles' block lookups at 2-8 blocks per 256 tokens."""
    announce(f"fused decode step {cache_dtype} cache, block {bs}")
    c = _case(dev, 100 + bs, 36, 16, 8, bs, torch.bfloat16, no_slot=(2,), cache_dtype=cache_dtype)
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float16])
def test_fused_decode_step_int32_lengths_and_wide_rows(dev, cache_dtype):
    """int32 context lengths, and qkv rows that are a slice of wider rows
    (a row stride of width + 136 elements)."""
    announce(f"fused decode step {cache_dtype} cache, int32 lengths, strided qkv")
    c = _case(dev, 77, 28, 32, 8, 16, torch.bfloat16, no_slot=(9,), cache_dtype=cache_dtype)
    c["ctx"] = c["ctx"].to(torch.int32)
    width = c["qkv"].shape[1]
    wide = torch.zeros(c["qkv"].shape[0], width + 136, dtype=c["qkv"].dtype, device=dev)
    wide[:, :width] = c["qkv"]
    c["qkv"] = wide[:, :width]
    assert c["qkv"].stride(0) == width + 136
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 8), (8, 8), (64, 8), (24, 3), (12, 4), (40, 8), (48, 8),
                                    (56, 8)])
@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.int8])
@pytest.mark.parametrize("bs", [16, 256])
def test_fused_decode_step_per_token_head_caches(dev, Hq, Hkv, cache_dtype, bs):
    """Per-token-head FP8 / INT8 caches: each appended row's scale from its
    head's amax (store_kv's), its codes, and the attention over tiles loaded
    after the append, except each wave's first tile, which goes out before
    it and is loaded again by the wave that holds the new token (the edge
    contexts of the first rows put it in a first tile); the codes, the
    per-slot scales and the output equal the two calls'."""
    announce(f"fused decode step per-token-head {cache_dtype} cache {Hq}/{Hkv} block {bs}")
    c = _case(dev, Hq * 3 + bs + 2, 40, Hq, Hkv, bs, torch.bfloat16, no_slot=(6, 33),
              cache_dtype=cache_dtype, per_token=True)
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("in_dtype", [torch.float16, torch.float32])
def test_fused_decode_step_16bit_cache_input_dtypes(dev, in_dtype):
    """An fp16 cache under fp16 / fp32 qkv rows (q in the rows' dtype)."""
    announce(f"fused decode step fp16 cache, {in_dtype} rows")
    c = _case(dev, 9, 24, 16, 8, 256, in_dtype, cache_dtype=torch.float16)
    _assert_same(_fused(c), _two_calls(c))


@pytest.mark.parametrize("in_dtype", [torch.float16, torch.float32])
def test_fused_decode_step_input_dtypes(dev, in_dtype):
    announce(f"fused decode step {in_dtype}")
    c = _case(dev, 5, 24, 16, 8, 256, in_dtype)
    _assert_same(_fused(c), _two_calls(c))


def test_fused_decode_step_engine_shape(dev):
    """The end-to-end engine's decode shape: 60 rows of 300-800 tokens,
    16 q / 8 kv heads, block 256, 4-block tables."""
    announce("fused decode step, engine shape")
    g = torch.Generator().manual_seed(11)
    ctx = torch.randint(300, 801, (60,), generator=g)
    c = _case(dev, 11, 60, 16, 8, 256, torch.bfloat16, ctx=ctx)
    _assert_same(_fused(c), _two_calls(c))


def test_fused_decode_step_large_batch(dev):
    """256 rows (0.5 M q elements): enough products and sums that an FMA the
    compiler fused in one of the two paths and not in the other would show
    (every product and sum is rounded on its own in both)."""
    announce("fused decode step, batch 256")
    g = torch.Generator().manual_seed(12)
    ctx = torch.randint(1, 801, (256,), generator=g)
    c = _case(dev, 12, 256, 16, 8, 256, torch.bfloat16, ctx=ctx, no_slot=(7, 100))
    _assert_same(_fused(c), _two_calls(c))


def test_fused_decode_step_calibrates_a_sentinel_scale(dev):
    """Scales still holding the 1.0 sentinel: the call calibrates them from
    its rows (every workgroup computes the same value), appends with them and
    attends with them, as the producer followed by the decode does."""
    announce("fused decode step, sentinel scales")
    c = _case(dev, 3, 20, 16, 8, 16, torch.bfloat16, scale_val=1.0)
    kc_u, vc_u = c["kc"].clone(), c["vc"].clone()
    ks_u, vs_u = c["ks"].clone(), c["vs"].clone()
    B, Hq, Hkv = c["B"], c["Hq"], c["Hkv"]
    q = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    _lib.call("mkv_qkv_norm_rope_append", c["qkv"].data_ptr(), c["qkv"].stride(0), _lib.DTYPE_BF16, B, Hq,
              Hkv, D, c["qw"].data_ptr(), c["kw"].data_ptr(), _lib.DTYPE_BF16, 1e-5, c["cs"].data_ptr(),
              _lib.DTYPE_BF16, c["cs"].shape[0], c["pos"].data_ptr(), q.data_ptr(), None, _lib.DTYPE_BF16,
              kc_u.data_ptr(), vc_u.data_ptr(), _lib.DTYPE_FP8E4M3, _lib.SCALE_PER_TENSOR, ks_u.data_ptr(),
              vs_u.data_ptr(), c["slots"].data_ptr(), c["bs"], kc_u.shape[0], _lib.APPEND_CALIBRATE_SENTINEL,
              A._stream(dev))
    out_u = A._decode(q, kc_u, vc_u, c["bt"], c["ctx"], c["scale"], Hq, Hkv, D, ks_u, vs_u,
                      split_tokens=A.DECODE_WORKGROUP)
    assert float(ks_u) != 1.0 and float(vs_u) != 1.0
    kc, vc = c["kc"].clone(), c["vc"].clone()
    ks, vs = c["ks"].clone(), c["vs"].clone()
    out = torch.empty_like(out_u)
    bt = c["bt"]
    _lib.call("mkv_qkv_norm_rope_append_decode", out.data_ptr(), out.stride(0), _lib.DTYPE_BF16,
              c["qkv"].data_ptr(), c["qkv"].stride(0), _lib.DTYPE_BF16, c["qw"].data_ptr(), c["kw"].data_ptr(),
              _lib.DTYPE_BF16, 1e-5, c["cs"].data_ptr(), _lib.DTYPE_BF16, c["cs"].shape[0], c["pos"].data_ptr(),
              kc.data_ptr(), vc.data_ptr(), _lib.DTYPE_FP8E4M3, kc.shape[0], ks.data_ptr(), vs.data_ptr(),
              _lib.SCALE_PER_TENSOR, c["slots"].data_ptr(), _lib.APPEND_CALIBRATE_SENTINEL, bt.data_ptr(),
              bt.stride(0), bt.shape[1], c["ctx"].data_ptr(), _lib.INDEX_I64, B, Hq, Hkv, D, c["bs"],
              c["scale"], A._stream(dev))
    _assert_same((out, kc, vc, ks, vs), (out_u, kc_u, vc_u, ks_u, vs_u))


@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 4)])
def test_fused_decode_step_matches_oracle(dev, Hq, Hkv):
    """The oracle's producer step (norm, rotary, FP8 append at the scales)
    and its decode over the dequantised cache; 2e-2 abs, the FP8 bound."""
    announce(f"fused decode step vs oracle {Hq}/{Hkv}")
    c = _case(dev, 17 + Hq, 30, Hq, Hkv, 16, torch.bfloat16, no_slot=(3,))
    out, kc, vc, ks, vs = _fused(c)
    qr, _, vr = R.qkv_norm_rope_ref(c["qkv"].cpu(), c["pos"].cpu(), Hq, Hkv, D, c["cs"].cpu(),
                                    c["qw"].cpu(), c["kw"].cpu(), 1e-5)
    # the appended V rows are the oracle's quantisation of the raw v
    slots = c["slots"].cpu()
    keep = slots >= 0
    v_codes = R.fp8_quantize_ref(vr[keep], float(c["vs"]))
    got = vc.cpu().reshape(-1, Hkv, D)[slots[keep]]
    assert torch.equal(got.view(torch.uint8), v_codes.view(torch.uint8))
    # (the K rows hold the kernel's rotated k, whose norm sums in another
    # order than the oracle's: the producer's own tests bound that)
    want = R.paged_decode_ref(qr, kc.cpu(), vc.cpu(), c["bt"].cpu(), c["ctx"].cpu(), c["scale"], Hq, Hkv,
                              k_scale=float(c["ks"]), v_scale=float(c["vs"]))
    assert_close_out(out, want, torch.bfloat16, 2e-2)
