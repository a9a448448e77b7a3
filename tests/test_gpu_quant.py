"""GPU parity of the per-token-head FP8 / INT8 modes (kv_cache_dtype
'fp8_per_token_head' and 'int8_per_token_head').

Append (reference attention.py:118-191, :194-276): codes and scales
bit-exact against the oracle, every byte of the pools and scale tensors
compared, including slots the append must not touch.

Decode (reference tile kernel attention.py:1124-1210): the oracle runs on the
very codes and scales the kernel reads, so the only difference is arithmetic:
2e-3 absolute plus half an output ulp (tighter than the 2e-2 allowed for FP8
KV against unquantised values).

Chunked prefill over the same caches (an extension; the reference's prefill
raises for quantised caches): the operator and the Attention layer's mixed
batch, against the oracle on the same codes and scales, within the FP8 KV
bound of 2e-2 (plus half an output ulp): the prefill kernel takes P times
the V scale as one fp16 MFMA operand (11 bits, as its per-tensor FP8 form
takes P), which leaves up to ~2^-12 |v| (3e-3 on these caches' |v| <= 16).
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import announce, assert_close_out
from mkv import attention as A
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu
FP8_MODE, INT8_MODE = "fp8_per_token_head", "int8_per_token_head"
CACHE_DT = {FP8_MODE: torch.float8_e4m3fn, INT8_MODE: torch.int8}
TOL = 2e-3
PREFILL_TOL = 2e-2


def _u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


def _rows(g, T, H, D, dtype):
    """Rows with per-(token, head) magnitudes spread over ~6 octaves, a few
    all-zero heads and a few NaN / inf elements."""
    x = torch.randn(T, H, D, generator=g) * torch.exp2(torch.rand(T, H, 1, generator=g) * 6 - 3)
    x[3, 1] = 0.0
    x[5, 0, 7] = float("nan")
    x[6, H - 1, 0] = -float("inf")
    return x.to(dtype)


def _append_both(dev, mode, key, value, slots, N, bs):
    H, D = key.shape[1], key.shape[2]
    cdt = CACHE_DT[mode]
    # pools and scales start from a marker pattern: untouched slots must keep it
    kc = torch.full((N, bs, H, D), 0x11, dtype=torch.uint8).view(cdt)
    vc = kc.clone()
    ks = torch.full((N, bs, H), 7.0)
    vs = torch.full((N, bs, H), 7.0)
    kr, vr, ksr, vsr = kc.clone(), vc.clone(), ks.clone(), vs.clone()
    kd, vd, ksd, vsd = kc.to(dev), vc.to(dev), ks.to(dev), vs.to(dev)
    if mode == INT8_MODE:
        A.store_kvcache_int8(key.to(dev), value.to(dev), kd, vd, ksd, vsd, slots.to(dev), bs)
    else:
        A.store_kvcache_fp8(key.to(dev), value.to(dev), kd, vd, ksd, vsd, slots.to(dev), bs, mode)
    R.store_kvcache_quant_ref(key.float(), value.float(), kr, vr, ksr, vsr, slots, mode)
    return (kd, vd, ksd, vsd), (kr, vr, ksr, vsr)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H,D", [(8, 128), (2, 64), (4, 256)])
def test_per_token_append_bit_exact(dev, mode, in_dtype, H, D):
    announce(f"append {mode}: {in_dtype} rows, {H} kv heads x {D}")
    seed = 10 * H + D + (500 if mode == INT8_MODE else 0) + \
        {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}[in_dtype]
    g = torch.Generator().manual_seed(seed)
    T, N, bs = 300, 40, 16
    key, value = _rows(g, T, H, D, in_dtype), _rows(g, T, H, D, in_dtype)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::7] = -1
    got, want = _append_both(dev, mode, key, value, slots, N, bs)
    for a, b in zip(got, want):
        assert torch.equal(_u8(a), b.view(torch.uint8))


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
def test_per_token_append_strided_rows(dev, mode):
    """K and V as views into a fused qkv buffer (row stride > row)."""
    announce(f"append {mode}: strided qkv views")
    g = torch.Generator().manual_seed(5)
    T, H, D, N, bs = 64, 8, 128, 8, 16
    qkv = (torch.randn(T, (32 + 2 * H) * D, generator=g) * 3).to(torch.bfloat16).to(dev)
    key = qkv[:, 32 * D:(32 + H) * D].view(T, H, D)
    value = qkv[:, (32 + H) * D:].view(T, H, D)
    assert key.stride(0) == (32 + 2 * H) * D
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    got, want = _append_both(dev, mode, key.cpu(), value.cpu(), slots, N, bs)
    for a, b in zip(got, want):
        assert torch.equal(_u8(a), b.view(torch.uint8))
    kc, vc, ks, vs = got
    kc2, vc2, ks2, vs2 = (t.clone().zero_() for t in got)
    if mode == INT8_MODE:
        A.store_kvcache_int8(key, value, kc2, vc2, ks2, vs2, slots.to(dev), bs)
    else:
        A.store_kvcache_fp8(key, value, kc2, vc2, ks2, vs2, slots.to(dev), bs, mode)
    for a, b in ((kc, kc2), (vc, vc2)):
        assert torch.equal(_u8(a).view(-1, H * D)[slots], _u8(b).view(-1, H * D)[slots])
    for a, b in ((ks, ks2), (vs, vs2)):
        assert torch.equal(a.cpu().view(-1, H)[slots], b.cpu().view(-1, H)[slots])


def _quant_pool(g, mode, N, bs, Hkv, D=128):
    k = torch.randn(N * bs, Hkv, D, generator=g) * torch.exp2(torch.rand(N * bs, Hkv, 1, generator=g) * 4 - 2)
    v = torch.randn(N * bs, Hkv, D, generator=g) * torch.exp2(torch.rand(N * bs, Hkv, 1, generator=g) * 4 - 2)
    kq, ks = R.quantize_per_token_head_ref(k.to(torch.bfloat16).float(), mode)
    vq, vs = R.quantize_per_token_head_ref(v.to(torch.bfloat16).float(), mode)
    return (kq.view(N, bs, Hkv, D), vq.view(N, bs, Hkv, D), ks.view(N, bs, Hkv),
            vs.view(N, bs, Hkv))


def _decode_case(seed, mode, B, Hq, Hkv, bs, N, max_blocks, ctx=None, qdt=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    if ctx is None:
        ctx = torch.randint(1, max_blocks * bs + 1, (B,), generator=g)
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=max_blocks)
    q = torch.randn(B, Hq, 128, generator=g).to(qdt)
    kq, vq, ks, vs = _quant_pool(g, mode, N, bs, Hkv)
    return q, kq, vq, ks, vs, bt, ctx.to(torch.int64)


def _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, scale, Hq, Hkv, split_tokens=0):
    out = A._decode(q.to(dev), kq.to(dev), vq.to(dev), bt.to(dev), ctx.to(dev), scale, Hq, Hkv,
                    128, ks.to(dev), vs.to(dev), split_tokens=split_tokens, per_token_head=True)
    return out.cpu()


def _oracle(q, kq, vq, ks, vs, bt, ctx, scale, Hq, Hkv):
    return R.paged_decode_ref(q.double(), kq, vq, bt, ctx, scale, Hq, Hkv, ks, vs)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("group", [1, 4, 8, 16])
@pytest.mark.parametrize("split_tokens", [0, 64, -1])
def test_per_token_decode_groups(dev, mode, group, split_tokens):
    announce(f"decode {mode}: group {group}, split_tokens {split_tokens}")
    Hkv = 2
    q, kq, vq, ks, vs, bt, ctx = _decode_case(200 + group, mode, 6, Hkv * group, Hkv, 32, 64, 10)
    got = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 1 / math.sqrt(128), Hkv * group, Hkv,
               split_tokens)
    want = _oracle(q, kq, vq, ks, vs, bt, ctx, 1 / math.sqrt(128), Hkv * group, Hkv)
    assert_close_out(got, want, got.dtype, TOL)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("bs", [16, 256])
def test_per_token_decode_edges(dev, mode, bs):
    """Context 0 / 1 / block edges, an absent block inside a context (its
    tokens are skipped, as in the other decode kernels; the reference's tile
    kernel would still count them in the denominator), padded rows with block
    entries 0 (graph replay), int32 and int64 context lengths."""
    announce(f"decode {mode}: bs {bs} edges")
    ctx = torch.tensor([0, 1, 2, bs - 1, bs, bs + 1, 3 * bs + 7, 31], dtype=torch.int64)
    q, kq, vq, ks, vs, bt, ctx = _decode_case(9 * bs, mode, 8, 8, 2, bs, 40, 5, ctx=ctx)
    bt[6, 1] = -1
    bt[0] = 0  # a padded graph row: context 0, table of zeros
    got = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 0.09, 8, 2)
    want = _oracle(q, kq, vq, ks, vs, bt, ctx, 0.09, 8, 2)
    assert_close_out(got, want, got.dtype, TOL)
    assert torch.count_nonzero(got[0]) == 0
    got32 = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx.to(torch.int32), 0.09, 8, 2)
    assert torch.equal(got, got32)
    # the same through the split-K kernel and the workgroup route
    got_sk = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 0.09, 8, 2, split_tokens=32)
    assert_close_out(got_sk, want, got.dtype, TOL)
    got_wg = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 0.09, 8, 2, split_tokens=-1)
    assert_close_out(got_wg, want, got.dtype, TOL)
    assert torch.count_nonzero(got_wg[0]) == 0


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("qdt", [torch.float32, torch.float16])
def test_per_token_decode_query_dtypes(dev, mode, qdt):
    """fp32 / fp16 queries: q is split into two bf16 terms (about 16 bits)."""
    announce(f"decode {mode}: {qdt} query")
    q, kq, vq, ks, vs, bt, ctx = _decode_case(77, mode, 3, 16, 4, 64, 40, 8, qdt=qdt)
    got = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 0.1, 16, 4)
    assert got.dtype == qdt
    want = _oracle(q, kq, vq, ks, vs, bt, ctx, 0.1, 16, 4)
    assert_close_out(got, want, got.dtype, TOL)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
def test_per_token_decode_uniform_scales_equal_per_tensor(dev, mode):
    """Codes in [-16, 16] are exact in both e4m3 and int8: with the same scale
    in every slot, the per-token-head kernel (bf16 MFMA) and the per-tensor
    FP8 kernel (fp16 MFMA) compute the same attention."""
    announce(f"decode {mode}: uniform scales vs per-tensor")
    g = torch.Generator().manual_seed(12)
    B, Hq, Hkv, bs, N, mb = 5, 16, 4, 32, 50, 8
    ctx = torch.randint(1, mb * bs + 1, (B,), generator=g)
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=mb)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16)
    codes = torch.randint(-16, 17, (2, N, bs, Hkv, 128), generator=g).float()
    kq = codes[0].to(CACHE_DT[mode])
    vq = codes[1].to(CACHE_DT[mode])
    ks = torch.full((N, bs, Hkv), 0.0625)
    vs = torch.full((N, bs, Hkv), 0.125)
    got = _run(dev, mode, q, kq, vq, ks, vs, bt, ctx, 0.1, Hq, Hkv)
    kf = codes[0].to(torch.float8_e4m3fn).to(dev)
    vf = codes[1].to(torch.float8_e4m3fn).to(dev)
    per_tensor = A.paged_attention_decode_quantized(
        q.to(dev), kf, vf, torch.tensor([0.0625], device=dev), torch.tensor([0.125], device=dev),
        bt.to(dev), ctx.to(dev), 0.1, Hq, Hkv, 128, bs, "fp8_per_tensor").cpu()
    want = _oracle(q, kq, vq, ks, vs, bt, ctx, 0.1, Hq, Hkv)
    assert_close_out(got, want, got.dtype, TOL)
    assert_close_out(per_tensor, want, got.dtype, TOL)


def _torch_gpu_reference_per_token(q, kc, vc, ks, vs, bt, ctx, scale, Hq, Hkv):
    """float32 torch reference on the GPU, one sequence at a time, with the
    per-slot scales applied to the gathered codes."""
    bs = kc.shape[1]
    G = Hq // Hkv
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for b in range(q.shape[0]):
        L = int(ctx[b])
        nb = (L + bs - 1) // bs
        blocks = bt[b, :nb].long()
        kk = (kc[blocks].float() * ks[blocks][..., None]).reshape(-1, Hkv, 128)[:L]
        vv = (vc[blocks].float() * vs[blocks][..., None]).reshape(-1, Hkv, 128)[:L]
        qq = q[b].float().reshape(Hkv, G, 128)
        s = torch.matmul(qq, kk.permute(1, 2, 0).contiguous()) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, vv.permute(1, 0, 2).contiguous()).reshape(Hq, 128)
    return out


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
def test_per_token_decode_batch256_full_size(dev, mode):
    announce(f"decode batch 256, 32/8 heads, ctx log-U[512, 8192], {mode}")
    m = W.decode_b256_metadata(seed=3)
    N, bs = m["num_blocks"], m["block_size"]
    kc = torch.empty(N, bs, 8, 128, dtype=CACHE_DT[mode], device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty(N, bs, 8, device=dev)
    vs = torch.empty_like(ks)
    W.fill_pools_per_token_head_on_device(kc, vc, ks, vs, 41, mode)
    g = torch.Generator().manual_seed(33)
    q = torch.randn(256, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    bt, ctx = m["block_tables"].to(dev), m["context_lens"].to(dev)
    got = A.paged_attention_decode_quantized(q, kc, vc, ks, vs, bt, ctx, 1 / math.sqrt(128), 32, 8,
                                             128, bs, mode)
    want = _torch_gpu_reference_per_token(q, kc, vc, ks, vs, bt, ctx, 1 / math.sqrt(128), 32, 8)
    assert_close_out(got, want, got.dtype, TOL)
    # deterministic run to run
    again = A.paged_attention_decode_quantized(q, kc, vc, ks, vs, bt, ctx, 1 / math.sqrt(128), 32,
                                               8, 128, bs, mode)
    assert torch.equal(got, again)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
def test_attention_layer_per_token_decode_step(dev, mode):
    """Attention.forward in a per-token-head mode: append the step's K/V,
    then decode, equal to calling the two operators by hand."""
    announce(f"Attention layer decode step, {mode}")
    from mkv import context as C
    g = torch.Generator().manual_seed(21)
    B, Hq, Hkv, bs, N, mb = 4, 16, 4, 16, 32, 6
    ctx = torch.tensor([5, 17, 40, 96], dtype=torch.int64)
    bt = W.fragmented_block_tables(ctx, bs, N, g, max_blocks=mb)
    slots = torch.tensor([int(bt[b, (int(ctx[b]) - 1) // bs]) * bs + (int(ctx[b]) - 1) % bs
                          for b in range(B)], dtype=torch.int64)
    kq, vq, ks, vs = (t.to(dev) for t in _quant_pool(g, mode, N, bs, Hkv))
    q = torch.randn(B, Hq, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, 128, generator=g).to(torch.bfloat16).to(dev)
    layer = A.Attention(Hq, 128, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    layer.k_cache, layer.v_cache = kq.clone(), vq.clone()
    layer.k_scale, layer.v_scale = ks.clone(), vs.clone()
    layer.kv_cache_dtype = mode
    C.set_context(False, slot_mapping=slots.to(dev), context_lens=ctx.to(dev),
                  block_tables=bt.to(dev))
    try:
        out = layer(q, k, v)
    finally:
        C.reset_context()
    kc2, vc2, ks2, vs2 = kq.clone(), vq.clone(), ks.clone(), vs.clone()
    if mode == INT8_MODE:
        A.store_kvcache_int8(k, v, kc2, vc2, ks2, vs2, slots.to(dev), bs)
    else:
        A.store_kvcache_fp8(k, v, kc2, vc2, ks2, vs2, slots.to(dev), bs, mode)
    want = A.paged_attention_decode_quantized(q, kc2, vc2, ks2, vs2, bt.to(dev), ctx.to(dev),
                                              1 / math.sqrt(128), Hq, Hkv, 128, bs, mode)
    assert torch.equal(out, want.reshape(B, Hq * 128))
    assert torch.equal(_u8(layer.k_cache), _u8(kc2)) and torch.equal(_u8(layer.v_scale), _u8(vs2))


# ---------------------------------------------------------------------------
# Chunked prefill over per-token-head caches (an extension: the reference's
# prefill raises for quantised caches, attention.py:1702-1708; the decode
# path's per-token arithmetic, attention.py:1124-1210, applied per key).
# ---------------------------------------------------------------------------
def _prefill_case(seed, mode, prior, qlen, Hq, Hkv, bs, qdt=torch.bfloat16, holes=()):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)], dtype=torch.int64)
    N = sum((int(c) + bs - 1) // bs for c in ctx) + 3
    bt = W.fragmented_block_tables(ctx, bs, N, g)
    for s, j in holes:
        bt[s, j] = -1
    cu = torch.zeros(len(qlen) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(qlen), 0).to(torch.int32)
    pos = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    q = torch.randn(int(cu[-1]), Hq, 128, generator=g).to(qdt)
    kq, vq, ks, vs = _quant_pool(g, mode, N, bs, Hkv)
    return q, kq, vq, ks, vs, bt, ctx, cu, pos


def _prefill_gpu(dev, mode, q, kq, vq, ks, vs, bt, ctx, cu, pos, scale, Hq, Hkv):
    out = A.paged_attention_prefill_triton(
        q.to(dev), kq.to(dev), vq.to(dev), bt.to(dev), ctx.to(dev), cu.to(dev), pos.to(dev), scale,
        Hq, Hkv, 128, kq.shape[1], k_scale=ks.to(dev), v_scale=vs.to(dev), kv_cache_dtype=mode)
    return out.cpu()


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("group", [1, 4, 16])
@pytest.mark.parametrize("qdt", [torch.bfloat16, torch.float32])
def test_per_token_prefill_matches_oracle(dev, mode, group, qdt):
    announce(f"per-token prefill {mode} group {group} q {qdt}")
    Hkv = 2
    q, kq, vq, ks, vs, bt, ctx, cu, pos = _prefill_case(30 + group, mode, [0, 37, 130, 5],
                                                        [70, 33, 1, 200], Hkv * group, Hkv, 32, qdt)
    sc = 1 / math.sqrt(128)
    got = _prefill_gpu(dev, mode, q, kq, vq, ks, vs, bt, ctx, cu, pos, sc, Hkv * group, Hkv)
    want = R.paged_prefill_ref(q.double(), kq, vq, bt, ctx, cu, pos, sc, Hkv * group, Hkv, ks, vs)
    assert_close_out(got, want, got.dtype, PREFILL_TOL)
    # and the arithmetic's own bound: one fp16 rounding of each P * v_scale
    # (2^-12 relative) weighs at most max |v|, taken here with a factor 2
    vmax = float((vq.float() * vs[..., None]).abs().max())
    assert_close_out(got, want, got.dtype, 2e-3 + 2.0 ** -11 * vmax)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("qdt,group", [(torch.bfloat16, 4), (torch.float32, 4), (torch.bfloat16, 16)])
def test_per_token_prefill_large_v_scales(dev, mode, qdt, group):
    """V scales 2^20 times the usual (V values of ~10^6): the prefill's P
    times the V scale is an fp16 MFMA operand, and a tile whose V scales
    would carry it past the fp16 maximum lifts the running max instead.
    The output is 2^20 times the unscaled one; divided back (exact for a
    power of two) it meets the oracle on the unscaled caches within the
    prefill bound."""
    announce(f"per-token prefill {mode} q {qdt} group {group}, V scales x 2^20")
    Hkv = 2
    q, kq, vq, ks, vs, bt, ctx, cu, pos = _prefill_case(60 + group, mode, [0, 400, 90], [130, 70, 200],
                                                        Hkv * group, Hkv, 16, qdt)
    sc = 1 / math.sqrt(128)
    S = float(2 ** 20)
    got = _prefill_gpu(dev, mode, q, kq, vq, ks, vs * S, bt, ctx, cu, pos, sc, Hkv * group, Hkv)
    assert torch.isfinite(got.float()).all()
    want = R.paged_prefill_ref(q.double(), kq, vq, bt, ctx, cu, pos, sc, Hkv * group, Hkv, ks, vs)
    assert_close_out(got / S, want, got.dtype, PREFILL_TOL)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("bs", [16, 256])
def test_per_token_prefill_block_sizes_holes_and_context_caps(dev, mode, bs):
    announce(f"per-token prefill {mode} bs {bs} holes")
    q, kq, vq, ks, vs, bt, ctx, cu, pos = _prefill_case(40 + bs, mode, [3, 0, 300], [129, 64, 17],
                                                        8, 2, bs, holes=[(2, 0)])
    ctx2 = ctx.clone()
    ctx2[0] = 50  # context shorter than some positions: visible = min(ctx, pos + 1)
    got = _prefill_gpu(dev, mode, q, kq, vq, ks, vs, bt, ctx2, cu, pos, 0.1, 8, 2)
    want = R.paged_prefill_ref(q.double(), kq, vq, bt, ctx2, cu, pos, 0.1, 8, 2, ks, vs)
    assert_close_out(got, want, got.dtype, PREFILL_TOL)


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
@pytest.mark.parametrize("route", ["unified", "split"])
def test_attention_layer_per_token_mixed_batch(dev, mode, route):
    """Attention.forward on a mixed batch (prefill chunks and decode rows,
    K/V already in the cache) in a per-token-head mode, both routes, against
    the oracle over every row."""
    announce(f"Attention layer per-token mixed batch, {mode}, {route}")
    from mkv import context as C
    Hq, Hkv, bs = 16, 4, 16
    prior, qlen = [40, 200, 7, 0, 120, 33], [1, 48, 1, 90, 1, 1]
    q, kq, vq, ks, vs, bt, ctx, cu, pos = _prefill_case(50, mode, prior, qlen, Hq, Hkv, bs)
    is_dec = [n == 1 for n in qlen]
    split = C.split_mixed_decode_prefill_metadata(cu.tolist(), qlen, is_dec)
    for name in ("decode_token_indices", "decode_seq_indices", "prefill_token_indices",
                 "prefill_seq_indices"):
        setattr(split, name + "_tensor", torch.tensor(getattr(split, name), device=dev))
    split.prefill_cu_seqlens_q_tensor = torch.tensor(split.prefill_cu_seqlens_q, dtype=torch.int32,
                                                     device=dev)
    layer = A.Attention(Hq, 128, scale=1.0, num_kv_heads=Hkv, block_size=bs)
    layer.k_cache, layer.v_cache = kq.to(dev), vq.to(dev)
    layer.k_scale, layer.v_scale = ks.to(dev), vs.to(dev)
    layer.kv_cache_dtype = mode
    layer.mixed_batch = route
    C.set_context(True, cu_seqlens_q=cu.to(dev), max_seqlen_q=max(qlen), slot_mapping=None,
                  context_lens=ctx.to(dev), block_tables=bt.to(dev), positions=pos.to(dev),
                  mixed_attention_split=split, is_full_prefill=False)
    try:
        qd = q.to(dev)
        out = layer(qd, qd, qd, kv_appended=True).cpu().view(-1, Hq, 128)
    finally:
        C.reset_context()
    want = R.paged_prefill_ref(q.double(), kq, vq, bt, ctx, cu, pos, 1 / math.sqrt(128), Hq, Hkv,
                               ks, vs)
    assert_close_out(out, want, out.dtype, PREFILL_TOL)
