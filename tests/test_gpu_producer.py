"""GPU parity of K6, the fused producer (q/k RMSNorm + rotary embedding + KV
append; reference qwen3.py:73-118, layernorm.py:16-24,
rotary_embedding.py:4-26, :100-109, attention.py:1654-1691).

* q and the rotated k against the oracle (qkv_norm_rope_ref): within four
  units in the last place of the output dtype at the head's largest
  element.  The
  kernel follows the reference's operation order (x / sqrt(mean + eps) *
  w, rounded to the input dtype, then x1*cos - x2*sin without fused
  multiply-adds), but its sum of squares adds in another order, so a
  normed value can land one rounding step away.
* The cache: bit-exact against the (separately pinned) append kernels run on
  the producer's own rotated k and the v view, for every cache format, so
  the fused append is exactly the unfused one.
"""
from __future__ import annotations

import pytest
import torch

from conftest import announce
from mkv import attention as A
from mkv import producer as P
from oracle import reference as R

pytestmark = pytest.mark.gpu
MANT = {torch.bfloat16: 8, torch.float16: 11, torch.float32: 24}


def _close_scaled(got, want, dtype, what):
    """|got - want| <= 4 ulp(dtype) * max |element| of the head + 1e-6: each
    output is x1*c - x2*s (or x1*s + x2*c), whose error follows the larger
    input of the pair even where the two terms cancel."""
    got, want = got.double().cpu(), want.double().cpu()
    scale = want.abs().amax(-1, keepdim=True).clamp(min=1e-3)
    tol = 4.0 * 2.0 ** (1 - MANT[dtype]) * scale + 1e-6
    err = (got - want).abs()
    # (a NaN difference fails unless both sides are NaN; `> tol` alone passes it)
    bad = ~(err <= tol) & ~(torch.isnan(got) & torch.isnan(want))
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} of {err.numel()} out of tolerance, max err {float(err.max()):.3e}"


def _inputs(seed, T, Hq, Hkv, D, in_dtype, cs_dtype, norm, max_pos=4096, extra_cols=0):
    g = torch.Generator().manual_seed(seed)
    width = (Hq + 2 * Hkv) * D
    qkv = (torch.randn(T, width + extra_cols, generator=g) * 2).to(in_dtype)
    pos = torch.randint(0, max_pos, (T,), generator=g)
    cs = R.rope_cos_sin_cache(1000000.0, D, max_pos).to(cs_dtype)
    qw = kw = None
    if norm:
        qw = (torch.rand(D, generator=g) + 0.5).to(in_dtype)
        kw = (torch.rand(D, generator=g) + 0.5).to(in_dtype)
    return qkv, pos, cs, qw, kw


@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cs_dtype", [torch.float32, "in"])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("Hq,Hkv,D", [(16, 8, 128), (8, 2, 64), (6, 2, 256)])
def test_producer_matches_oracle_copy_cache(dev, in_dtype, cs_dtype, norm, Hq, Hkv, D):
    cs_dtype = in_dtype if cs_dtype == "in" else cs_dtype
    announce(f"producer {in_dtype} cos_sin {cs_dtype} norm {norm} {Hq}/{Hkv}x{D}")
    T, N, bs = 200, 30, 16
    qkv, pos, cs, qw, kw = _inputs(Hq * D + int(norm), T, Hq, Hkv, D, in_dtype, cs_dtype, norm)
    slots = torch.randperm(N * bs, generator=torch.Generator().manual_seed(1))[:T].to(torch.int64)
    slots[::9] = -1
    kc = torch.zeros(N, bs, Hkv, D, dtype=in_dtype, device=dev)
    vc = torch.zeros_like(kc)
    q, k, v = P.qkv_norm_rope_append(qkv.to(dev), pos.to(dev), Hq, Hkv, D, cs.to(dev), kc, vc,
                                     slots.to(dev), bs, q_norm_weight=None if qw is None else qw.to(dev),
                                     k_norm_weight=None if kw is None else kw.to(dev), return_k=True)
    qr, kr, vr = R.qkv_norm_rope_ref(qkv, pos, Hq, Hkv, D, cs, qw, kw, 1e-5)
    _close_scaled(q, qr, in_dtype, "q")
    _close_scaled(k, kr, in_dtype, "k")
    assert torch.equal(v.cpu(), vr)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    A.store_kvcache(k, v, kc2, vc2, slots.to(dev), bs)
    assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8))


@pytest.mark.parametrize("mode", ["fp8_per_tensor", "fp8_per_token_head", "int8_per_token_head"])
def test_producer_quantised_caches_equal_unfused_append(dev, mode):
    announce(f"producer {mode}: fused append == unfused append of its k / v")
    T, Hq, Hkv, D, N, bs = 300, 16, 8, 128, 40, 16
    cdt = torch.int8 if mode == "int8_per_token_head" else torch.float8_e4m3fn
    per_token = mode != "fp8_per_tensor"

    def fresh():
        kc = torch.zeros(N, bs, Hkv, D, dtype=cdt, device=dev)
        shape = (N, bs, Hkv) if per_token else (1,)
        return kc, torch.zeros_like(kc), torch.ones(shape, device=dev), torch.ones(shape, device=dev)

    kc, vc, ks, vs = fresh()
    for call in range(2):  # per tensor: the first call calibrates, the second is fused
        qkv, pos, cs, qw, kw = _inputs(90 + call, T, Hq, Hkv, D, torch.bfloat16, torch.float32, True)
        slots = torch.randperm(N * bs, generator=torch.Generator().manual_seed(call))[:T].to(torch.int64)
        slots[::11] = -1
        args = (qkv.to(dev), pos.to(dev), Hq, Hkv, D, cs.to(dev))
        kw_ = dict(q_norm_weight=qw.to(dev), k_norm_weight=kw.to(dev), kv_cache_dtype=mode,
                   k_scale=ks, v_scale=vs, return_k=True)
        before = (kc.clone(), vc.clone(), ks.clone(), vs.clone())
        q, k, v = P.qkv_norm_rope_append(*args, kc, vc, slots.to(dev), bs, **kw_)
        kc2, vc2, ks2, vs2 = (t.clone() for t in before)
        if not per_token:
            A.calibrate_fp8_per_tensor(k, v, ks2, vs2)
        if mode == "int8_per_token_head":
            A.store_kvcache_int8(k, v, kc2, vc2, ks2, vs2, slots.to(dev), bs)
        elif per_token:
            A.store_kvcache_fp8(k, v, kc2, vc2, ks2, vs2, slots.to(dev), bs, mode)
        else:
            A._append(k, v, kc2, vc2, slots.to(dev), ks2, vs2)
        for a, b in ((kc, kc2), (vc, vc2), (ks, ks2), (vs, vs2)):
            assert torch.equal(a.cpu().view(torch.uint8), b.cpu().view(torch.uint8)), f"call {call}"
        qr, kr, _ = R.qkv_norm_rope_ref(qkv, pos, Hq, Hkv, D, cs, qw, kw, 1e-5)
        _close_scaled(q, qr, torch.bfloat16, "q")
        _close_scaled(k, kr, torch.bfloat16, "k")
    if not per_token:
        assert ks._mkv_calibrated and float(ks) != 1.0


def test_producer_per_tensor_sentinel_fallback(dev):
    """A per-tensor scale reset to 1.0 after its first use is calibrated by
    the fused kernel itself, from this call's rotated k (all rows)."""
    announce("producer fp8 per-tensor sentinel fallback")
    T, Hq, Hkv, D, N, bs = 64, 8, 4, 128, 12, 16
    qkv, pos, cs, qw, kw = _inputs(95, T, Hq, Hkv, D, torch.bfloat16, torch.float32, True)
    slots = torch.randperm(N * bs, generator=torch.Generator().manual_seed(3))[:T].to(torch.int64)
    slots[0] = -1
    kc = torch.zeros(N, bs, Hkv, D, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks, vs = torch.ones(1, device=dev), torch.ones(1, device=dev)
    args = (qkv.to(dev), pos.to(dev), Hq, Hkv, D, cs.to(dev))
    kw_ = dict(q_norm_weight=qw.to(dev), k_norm_weight=kw.to(dev), kv_cache_dtype="fp8_per_tensor",
               k_scale=ks, v_scale=vs, return_k=True)
    P.qkv_norm_rope_append(*args, kc, vc, slots.to(dev), bs, **kw_)
    first = (float(ks), float(vs))
    ks.fill_(1.0)
    vs.fill_(1.0)
    kc.zero_()
    vc.zero_()
    q, k, v = P.qkv_norm_rope_append(*args, kc, vc, slots.to(dev), bs, **kw_)
    assert (float(ks), float(vs)) == first
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    A._append(k, v, kc2, vc2, slots.to(dev), ks, vs)
    assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8))


def test_producer_strided_rows_and_out_of_range_position(dev):
    announce("producer: strided qkv rows, fp32 out, a position past the table")
    T, Hq, Hkv, D, N, bs, P_max = 40, 8, 2, 128, 8, 16, 64
    qkv, pos, cs, qw, kw = _inputs(96, T, Hq, Hkv, D, torch.bfloat16, torch.float32, True,
                                   max_pos=P_max, extra_cols=64)
    pos[7] = P_max  # outside the table: that row's q / k are NaN, nothing else changes
    qkv_d = qkv.to(dev)
    assert qkv_d.stride(0) > (Hq + 2 * Hkv) * D
    slots = torch.arange(T, dtype=torch.int64)
    kc = torch.zeros(N, bs, Hkv, D, dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    q, k, v = P.qkv_norm_rope_append(qkv_d, pos.to(dev), Hq, Hkv, D, cs.to(dev), kc, vc, slots.to(dev),
                                     bs, q_norm_weight=qw.to(dev), k_norm_weight=kw.to(dev),
                                     out_dtype=torch.float32, return_k=True)
    assert q.dtype == torch.float32 and bool(torch.isnan(q[7]).all()) and bool(torch.isnan(k[7]).all())
    ok = torch.ones(T, dtype=torch.bool)
    ok[7] = False
    qr, kr, _ = R.qkv_norm_rope_ref(qkv[:, :(Hq + 2 * Hkv) * D][ok], pos[ok], Hq, Hkv, D, cs, qw, kw,
                                    1e-5, out_dtype=torch.float32)
    # the normed values are rounded to the bf16 input dtype before the rotation
    _close_scaled(q[ok.to(dev)], qr, torch.bfloat16, "q")
    _close_scaled(k[ok.to(dev)], kr, torch.bfloat16, "k")


def test_attention_layer_after_the_fused_producer(dev):
    """Producer + Attention(kv_appended=True) equals the reference's order:
    norm + rotary in torch-on-GPU, then Attention.forward storing and
    attending (decode step, FP8 per-tensor cache)."""
    announce("producer + Attention(kv_appended=True) decode step")
    from mkv import context as C
    g = torch.Generator().manual_seed(97)
    B, Hq, Hkv, D, bs, N = 6, 16, 8, 128, 16, 48
    ctx = torch.tensor([5, 17, 33, 48, 70, 100], dtype=torch.int64)
    bt = torch.arange(N, dtype=torch.int32)[:42].view(B, 7)
    slots = torch.tensor([int(bt[b, (int(ctx[b]) - 1) // bs]) * bs + (int(ctx[b]) - 1) % bs
                          for b in range(B)], dtype=torch.int64)
    qkv, pos, cs, qw, kw = _inputs(98, B, Hq, Hkv, D, torch.bfloat16, torch.bfloat16, True)
    pos = ctx - 1
    prior = torch.randn(N * bs, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
    outs = []
    for fused in (True, False):
        kc = torch.zeros(N, bs, Hkv, D, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.zeros_like(kc)
        ks, vs = torch.full((1,), 0.03, device=dev), torch.full((1,), 0.03, device=dev)
        A._append(prior, prior, kc, vc, torch.arange(N * bs, device=dev), ks, vs)
        layer = A.Attention(Hq, D, scale=1.0, num_kv_heads=Hkv, block_size=bs)
        layer.k_cache, layer.v_cache, layer.k_scale, layer.v_scale = kc, vc, ks, vs
        layer.kv_cache_dtype = "fp8_per_tensor"
        C.set_context(False, slot_mapping=slots.to(dev), context_lens=ctx.to(dev), block_tables=bt.to(dev))
        try:
            if fused:
                q, k, v = P.qkv_norm_rope_append(
                    qkv.to(dev), pos.to(dev), Hq, Hkv, D, cs.to(dev), kc, vc, slots.to(dev), bs,
                    q_norm_weight=qw.to(dev), k_norm_weight=kw.to(dev), kv_cache_dtype="fp8_per_tensor",
                    k_scale=ks, v_scale=vs)
                o = layer(q, k, v, kv_appended=True)
            else:
                q, k, v = P.qkv_norm_rope_append(
                    qkv.to(dev), pos.to(dev), Hq, Hkv, D, cs.to(dev), None, None, None, bs,
                    q_norm_weight=qw.to(dev), k_norm_weight=kw.to(dev), return_k=True)
                o = layer(q, k, v.contiguous())
        finally:
            C.reset_context()
        outs.append((o, kc.clone(), vc.clone()))
    (o1, k1, v1), (o2, k2, v2) = outs
    assert torch.equal(k1.view(torch.uint8), k2.view(torch.uint8))
    assert torch.equal(v1.view(torch.uint8), v2.view(torch.uint8))
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
