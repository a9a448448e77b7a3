"""Pins for the CPU oracle (oracle/), run on the CPU.

The reference ships no golden vectors for this path, so each oracle function
is pinned by something it does not itself compute: the format definition of
e4m3fn, closed forms and known answers, invariants that a dropped term or a
wrong index would break, and the literal loop restatements of the reference
kernels in float64 (plus the committed fixtures under tests/golden/).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import fp8_codec
from oracle import reference as R

# ---------------------------------------------------------------------------
# FP8 e4m3fn: torch's cast against the format definition
# ---------------------------------------------------------------------------


def test_fp8_decode_table_matches_format_definition():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    t = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ref = fp8_codec.decode_e4m3fn(codes.numpy())
    assert np.array_equal(np.isnan(t), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(t[ok], ref[ok])
    # spot values from the definition
    assert ref[0x7E] == 448.0 and ref[0x01] == 2.0 ** -9 and ref[0x08] == 2.0 ** -6
    assert np.isnan(ref[0x7F]) and np.isnan(ref[0xFF])


def _torch_bytes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_fp8_encode_all_bf16_patterns():
    # every bf16 bit pattern, as float32, clamped like the reference
    bits = np.arange(65536, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    xc = np.where(np.isnan(x), x, np.clip(x, -448.0, 448.0)).astype(np.float32)
    assert np.array_equal(_torch_bytes(xc), fp8_codec.encode_e4m3fn(xc))


def test_fp8_encode_random_fp32_and_ties():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * np.exp2(rng.integers(-14, 9, 200_000))).astype(np.float32)
    x = np.clip(x, -448, 448).astype(np.float32)
    # exact midpoints between adjacent codes (ties to even) and their neighbours
    vals = fp8_codec.decode_e4m3fn(np.arange(0x7F, dtype=np.uint8))
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    edge = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                           -mids, np.float32([0.0, -0.0, 448.0, -448.0, 2.0 ** -10, 3 * 2.0 ** -11])])
    for arr in (x, edge.astype(np.float32)):
        assert np.array_equal(_torch_bytes(arr), fp8_codec.encode_e4m3fn(arr))


def test_fp8_quantize_ref_equals_codec():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4096, generator=g) * 30).to(torch.bfloat16)
    for scale in (1.0, 0.0123, 0.25, 3.5, 448.0 / 7):
        got = R.fp8_quantize_ref(x, scale).view(torch.uint8).numpy()
        want = fp8_codec.quantize_per_tensor(x.float().numpy(), scale)
        assert np.array_equal(got, want)
    # saturation: values beyond 448*scale clamp to +-448 (0x7e / 0xfe), never NaN
    big = torch.tensor([1e4, -1e4, 449.0, -500.0], dtype=torch.float32)
    assert R.fp8_quantize_ref(big, 1.0).view(torch.uint8).tolist() == [0x7E, 0xFE, 0x7E, 0xFE]


# ---------------------------------------------------------------------------
# Per-tensor calibration (attention.py:318-323)
# ---------------------------------------------------------------------------


def _rule(amax: float, dtype: torch.dtype) -> float:
    """round_in(max(round_in(amax), round_in(1e-8)) / 448): the rule the
    device kernel implements, written with explicit roundings."""
    def rnd(v):
        return float(torch.tensor(v, dtype=torch.float32).to(dtype).float())
    a = max(rnd(amax), rnd(1e-8))
    return rnd(float(np.float32(a) / np.float32(448.0)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_calibration_rule_matches_torch_expression(dtype):
    # all positive bf16 / f16 values (or a dense fp32 sample) as amax
    if dtype == torch.bfloat16:
        vals = (np.arange(0, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    elif dtype == torch.float16:
        vals = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    else:
        rng = np.random.default_rng(1)
        vals = np.abs(rng.standard_normal(20000).astype(np.float32) * np.exp2(rng.integers(-30, 30, 20000))).astype(np.float32)
    xs = torch.from_numpy(vals.astype(np.float32)).to(dtype)
    got = (xs.abs().clamp(min=1e-8) / 448.0).float()  # torch evaluates elementwise in dtype
    for i in range(0, len(vals), max(1, len(vals) // 3000)):
        assert float(got[i]) == _rule(float(xs[i].float()), dtype), (dtype, float(xs[i]))


def test_calibration_known_answers():
    # amax 448 -> scale exactly 1.0 (which the reference would re-calibrate next call)
    x = torch.zeros(4, 8, dtype=torch.bfloat16)
    x[1, 3] = -448.0
    assert R.calibrate_scale_ref(x) == 1.0
    # all-zero bf16 input -> the bf16 rounding of 1e-8 divided by 448 in bf16
    z = torch.zeros(3, 5, dtype=torch.bfloat16)
    want = float(torch.tensor(float(torch.tensor(1e-8, dtype=torch.bfloat16)) / 448.0).to(torch.bfloat16))
    assert R.calibrate_scale_ref(z) == want
    # fp16 cannot represent 1e-8: the clamp floor rounds to 0, so the scale is 0
    assert R.calibrate_scale_ref(torch.zeros(2, 2, dtype=torch.float16)) == 0.0
    # bf16 rounding of amax / 448 (amax = 20 -> 0.044642857 -> bf16 0.044677734375)
    y = torch.tensor([[20.0, -3.0]], dtype=torch.bfloat16)
    assert R.calibrate_scale_ref(y) == float(torch.tensor(20.0 / 448.0).to(torch.bfloat16))


def test_store_kvcache_fp8_ref_calibrates_once_and_skips_padding():
    g = torch.Generator().manual_seed(3)
    T, H, D, N, bs = 10, 2, 16, 4, 8
    k = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    k[7] *= 50  # the amax row is a padding row: it must still count
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[7] = -1
    kc = torch.zeros(N, bs, H, D, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1)
    vs = torch.ones(1)
    R.store_kvcache_fp8_ref(k, v, kc, vc, ks, vs, slots)
    assert float(ks) == R.calibrate_scale_ref(k) and float(ks) == float(
        (k.abs().amax() / 448.0).to(torch.bfloat16))
    first = float(ks)
    R.store_kvcache_fp8_ref(k * 2, v, kc, vc, ks, vs, slots)  # frozen after first calibration
    assert float(ks) == first
    # untouched slots stay zero; written slots hold the codec's bytes
    flat = kc.view(-1, H, D).view(torch.uint8)
    written = set(slots[slots >= 0].tolist())
    for s in range(N * bs):
        if s not in written:
            assert int(flat[s].sum()) == 0
    t = 3
    want = fp8_codec.quantize_per_tensor((k[t] * 2).float().numpy(), first)
    assert np.array_equal(flat[int(slots[t])].numpy(), want)


def test_store_kvcache_ref_matches_loop():
    g = torch.Generator().manual_seed(4)
    T, H, D, N, bs = 12, 3, 16, 5, 4
    k = torch.randn(T, H, D, generator=g)
    v = torch.randn(T, H, D, generator=g)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::5] = -1
    kc, vc = torch.zeros(N, bs, H, D), torch.zeros(N, bs, H, D)
    R.store_kvcache_ref(k, v, kc, vc, slots)
    kl, vl = torch.zeros(N, bs, H, D), torch.zeros(N, bs, H, D)
    for t in range(T):
        s = int(slots[t])
        if s == -1:
            continue
        kl[s // bs, s % bs] = k[t]
        vl[s // bs, s % bs] = v[t]
    assert torch.equal(kc, kl) and torch.equal(vc, vl)


# ---------------------------------------------------------------------------
# Decode oracle
# ---------------------------------------------------------------------------


def _tiny_decode(seed, B=2, Hq=4, Hkv=2, D=16, N=12, bs=8, max_blocks=5, fp8=False):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_blocks * bs + 1, (B,), generator=g)
    perm = torch.randperm(N, generator=g)
    bt = torch.full((B, max_blocks), -1, dtype=torch.int32)
    pos = 0
    for b in range(B):
        nb = (int(ctx[b]) + bs - 1) // bs
        bt[b, :nb] = perm[pos:pos + nb].to(torch.int32) if pos + nb <= N else perm[:nb].to(torch.int32)
        pos += nb
    q = torch.randn(B, Hq, D, generator=g)
    k = torch.randn(N, bs, Hkv, D, generator=g)
    v = torch.randn(N, bs, Hkv, D, generator=g)
    ks = vs = None
    if fp8:
        ks, vs = R.calibrate_scale_ref(k), R.calibrate_scale_ref(v)
        k, v = R.fp8_quantize_ref(k, ks), R.fp8_quantize_ref(v, vs)
    return q, k, v, bt, ctx, ks, vs


@pytest.mark.parametrize("seed,fp8", [(0, False), (1, False), (2, True), (3, True)])
def test_decode_ref_matches_literal_loops(seed, fp8):
    q, k, v, bt, ctx, ks, vs = _tiny_decode(seed, fp8=fp8)
    scale = 0.25
    got = R.paged_decode_ref(q, k, v, bt, ctx, scale, 4, 2, ks, vs)
    want = R.paged_decode_literal(q, k, v, bt, ctx, scale, 4, 2, ks, vs)
    assert torch.allclose(got.double(), want, atol=1e-6, rtol=0)


def test_decode_ref_matches_sdpa_on_identity_tables():
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, D, bs, nb = 3, 8, 2, 16, 4, 5
    q = torch.randn(B, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(B * nb, bs, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(B * nb, bs, Hkv, D, generator=g, dtype=torch.float64)
    bt = torch.arange(B * nb, dtype=torch.int32).reshape(B, nb)
    L = nb * bs
    ctx = torch.full((B,), L, dtype=torch.int64)
    got = R.paged_decode_ref(q, k, v, bt, ctx, 0.3, Hq, Hkv)
    kk = k.reshape(B, L, Hkv, D).repeat_interleave(Hq // Hkv, dim=2).transpose(1, 2)
    vv = v.reshape(B, L, Hkv, D).repeat_interleave(Hq // Hkv, dim=2).transpose(1, 2)
    want = torch.nn.functional.scaled_dot_product_attention(q[:, :, None], kk, vv, scale=0.3)[:, :, 0]
    assert torch.allclose(got, want, atol=1e-12)


def test_decode_ref_invariants():
    q, k, v, bt, ctx, _, _ = _tiny_decode(11)
    base = R.paged_decode_ref(q, k, v, bt, ctx, 0.5, 4, 2)
    # permuting physical blocks together with the tables changes nothing
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.argsort(perm)
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].to(torch.int32), bt)
    out2 = R.paged_decode_ref(q, k[perm], v[perm], bt2, ctx, 0.5, 4, 2)
    assert torch.allclose(base, out2, atol=1e-12)
    # extra -1 padding columns change nothing
    bt3 = torch.cat([bt, torch.full((bt.shape[0], 3), -1, dtype=torch.int32)], 1)
    assert torch.allclose(base, R.paged_decode_ref(q, k, v, bt3, ctx, 0.5, 4, 2), atol=1e-12)
    # context 1 -> V of token 0; constant K -> mean of V
    one = torch.ones_like(ctx)
    o1 = R.paged_decode_ref(q, k, v, bt, one, 0.5, 4, 2)
    for b in range(q.shape[0]):
        p = int(bt[b, 0])
        assert torch.allclose(o1[b].reshape(2, 2, -1), v[p, 0][:, None, :].expand(2, 2, -1), atol=1e-12)
    kc = torch.ones_like(k)
    oc = R.paged_decode_ref(q, kc, v, bt, ctx, 0.5, 4, 2)
    for b in range(q.shape[0]):
        L = int(ctx[b])
        rows = torch.stack([v[int(bt[b, t // 8]), t % 8] for t in range(L)])
        assert torch.allclose(oc[b].reshape(2, 2, -1), rows.mean(0)[:, None, :].expand(2, 2, -1), atol=1e-6)
    # zero context -> zeros
    assert torch.count_nonzero(R.paged_decode_ref(q, k, v, bt, torch.zeros_like(ctx), 0.5, 4, 2)) == 0


def test_decode_torch_optimized_matches_ref():
    q, k, v, bt, ctx, _, _ = _tiny_decode(21)
    bt_full = bt.clone()
    a = R.decode_torch_optimized_ref(q, k, v, bt_full, ctx, 0.5, 4, 2, 16, 8)
    b = R.paged_decode_ref(q, k, v, bt, ctx, 0.5, 4, 2)
    assert torch.allclose(a, b, atol=1e-5)
    c = R.decode_torch_optimized_ref(q, k, v, bt_full, ctx, 0.5, 4, 2, 16, 8, micro_batch=1)
    assert torch.allclose(a, c, atol=1e-6)


# ---------------------------------------------------------------------------
# Prefill oracle
# ---------------------------------------------------------------------------


def _tiny_prefill(seed, fp8=False, Hq=4, Hkv=2, D=16, bs=8, N=20):
    g = torch.Generator().manual_seed(seed)
    prior = [0, 5, 11]
    qlen = [7, 4, 1]
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)], dtype=torch.int64)
    perm = torch.randperm(N, generator=g)
    nbs = [(int(c) + bs - 1) // bs for c in ctx]
    bt = torch.full((3, max(nbs)), -1, dtype=torch.int32)
    pos = 0
    for s, nb in enumerate(nbs):
        bt[s, :nb] = perm[pos:pos + nb].to(torch.int32)
        pos += nb
    cu = torch.tensor([0] + list(np.cumsum(qlen)), dtype=torch.int32)
    positions = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    q = torch.randn(int(cu[-1]), Hq, D, generator=g)
    k = torch.randn(N, bs, Hkv, D, generator=g)
    v = torch.randn(N, bs, Hkv, D, generator=g)
    ks = vs = None
    if fp8:
        ks, vs = R.calibrate_scale_ref(k), R.calibrate_scale_ref(v)
        k, v = R.fp8_quantize_ref(k, ks), R.fp8_quantize_ref(v, vs)
    return q, k, v, bt, ctx, cu, positions, ks, vs


@pytest.mark.parametrize("seed,fp8", [(0, False), (1, True)])
def test_prefill_ref_matches_literal(seed, fp8):
    q, k, v, bt, ctx, cu, pos, ks, vs = _tiny_prefill(seed, fp8)
    got = R.paged_prefill_ref(q, k, v, bt, ctx, cu, pos, 0.3, 4, 2, ks, vs)
    want = R.paged_prefill_literal(q, k, v, bt, ctx, cu, pos, 0.3, 4, 2, ks, vs)
    assert torch.allclose(got.double(), want, atol=1e-6)


def test_prefill_ref_special_cases():
    q, k, v, bt, ctx, cu, pos, _, _ = _tiny_prefill(5)
    out = R.paged_prefill_ref(q, k, v, bt, ctx, cu, pos, 0.3, 4, 2)
    # the single-row sequence (q_len 1 at position ctx-1) equals decode
    s = 2
    r = int(cu[s])
    dec = R.paged_decode_ref(q[r:r + 1], k, v, bt[s:s + 1], ctx[s:s + 1], 0.3, 4, 2)
    assert torch.allclose(out[r:r + 1], dec, atol=1e-6)
    # sequence 0 starts at position 0: equals causal attention over its own rows
    n = int(cu[1])
    rows = torch.stack([k[int(bt[0, t // 8]), t % 8] for t in range(n)])
    vrow = torch.stack([v[int(bt[0, t // 8]), t % 8] for t in range(n)])
    full = R.flash_prefill_ref(q[:n], rows, vrow, torch.tensor([0, n]), 0.3, 4, 2)
    assert torch.allclose(out[:n], full, atol=1e-6)
    # splitting a sequence's rows into chunks (same positions) changes nothing
    cu2 = torch.tensor([0, 3, 7, 11, 12], dtype=torch.int32)
    ctx2 = torch.tensor([3, 7, 16, 12], dtype=torch.int64)
    bt2 = torch.cat([bt[:1], bt[:1], bt[1:]])
    out2 = R.paged_prefill_ref(q, k, v, bt2, ctx2, cu2, pos, 0.3, 4, 2)
    assert torch.allclose(out, out2, atol=1e-6)


def test_flash_prefill_ref_matches_sdpa():
    g = torch.Generator().manual_seed(9)
    Hq, Hkv, D = 4, 2, 16
    lens = [5, 1, 9]
    cu = torch.tensor([0, 5, 6, 15], dtype=torch.int32)
    q = torch.randn(15, Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(15, Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(15, Hkv, D, generator=g, dtype=torch.float64)
    got = R.flash_prefill_ref(q, k, v, cu, 0.2, Hq, Hkv)
    for s, n in enumerate(lens):
        a = int(cu[s])
        qq = q[a:a + n].transpose(0, 1)[None]
        kk = k[a:a + n].transpose(0, 1).repeat_interleave(2, 0)[None]
        vv = v[a:a + n].transpose(0, 1).repeat_interleave(2, 0)[None]
        want = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True, scale=0.2)
        assert torch.allclose(got[a:a + n], want[0].transpose(0, 1), atol=1e-12)


def test_gather_ref():
    q, k, v, bt, ctx, _, _ = _tiny_decode(31)
    out = R.gather_kv_ref(k, bt, ctx, 40)
    for b in range(bt.shape[0]):
        for t in range(40):
            if t < int(ctx[b]):
                assert torch.equal(out[b, t], k[int(bt[b, t // 8]), t % 8])
            else:
                assert int(torch.count_nonzero(out[b, t])) == 0


# ---------------------------------------------------------------------------
# Per-token-head FP8 / INT8 quantisation (attention.py:166-181, :194-243)
# ---------------------------------------------------------------------------
FP8_MODE, INT8_MODE = "fp8_per_token_head", "int8_per_token_head"


def test_per_token_fp8_known_answers():
    g = torch.Generator().manual_seed(31)
    x = torch.randn(5, 3, 16, generator=g) * 100
    # amax exactly 448 -> scale exactly 1 -> the codes are torch's own cast
    x[..., 3] = 448.0
    q, s = R.quantize_per_token_head_ref(x, FP8_MODE)
    assert torch.equal(s, torch.ones(5, 3))
    assert torch.equal(q.view(torch.uint8), x.to(torch.float8_e4m3fn).view(torch.uint8))
    # an all-zero head -> scale 1 and zero codes; NaN elements do not count
    # towards amax and stay NaN
    z = torch.zeros(1, 2, 16)
    z[0, 1, 0], z[0, 1, 5] = float("nan"), -2.0
    q, s = R.quantize_per_token_head_ref(z, FP8_MODE)
    assert float(s[0, 0]) == 1.0 and torch.count_nonzero(q[0, 0].view(torch.uint8)) == 0
    assert float(s[0, 1]) == np.float32(2.0) / np.float32(448.0)
    assert int(q[0, 1, 5].view(torch.uint8)) == 0xFE  # -448
    assert int(q[0, 1, 0].view(torch.uint8)) & 0x7F == 0x7F  # NaN


def test_per_token_fp8_power_of_two_invariance_and_error_bound():
    g = torch.Generator().manual_seed(32)
    x = torch.randn(7, 4, 64, generator=g) * torch.rand(7, 4, 1, generator=g) * 10
    q, s = R.quantize_per_token_head_ref(x, FP8_MODE)
    for k in (-5, 3, 11):
        q2, s2 = R.quantize_per_token_head_ref(x * 2.0 ** k, FP8_MODE)
        assert torch.equal(s2, s * 2.0 ** k)
        assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8))
    # the head's amax maps to +-448 and every element is within half an e4m3
    # step (3 mantissa bits) of x / scale, or below the subnormal step
    y = x / s[..., None]
    deq = q.to(torch.float64)
    amax_pos = x.abs().argmax(dim=-1, keepdim=True)
    assert torch.equal(deq.abs().gather(-1, amax_pos), torch.full_like(deq[..., :1], 448.0))
    step = torch.exp2(torch.floor(torch.log2(y.abs().clamp(min=2.0 ** -6))) - 3)
    assert bool(((deq - y.double()).abs() <= step.double() / 2 + 1e-12).all())


def test_per_token_int8_known_answers():
    # amax 127 -> scale 1, 1 / scale 1: the rounding is half away from zero
    x = torch.tensor([2.5, -2.5, 0.49, -0.5, 126.6, -127.0, 1.5, -1.49, 127.0, 0.5,
                      -0.0, 3.0, -3.5, 60.5, -60.5, 0.0]).reshape(1, 1, 16)
    q, s = R.quantize_per_token_head_ref(x, INT8_MODE)
    assert float(s) == 1.0
    assert q.flatten().tolist() == [3, -3, 0, -1, 127, -127, 2, -1, 127, 1, 0, 3, -4, 61, -61, 0]
    # an all-zero head -> scale 1e-6 (fp32) and zero codes; a tiny head is
    # floored at 1e-6 too; a NaN becomes -128 and does not count towards amax
    z = torch.zeros(3, 1, 16)
    z[1, 0, :2] = torch.tensor([1e-5, -4e-6])
    z[2, 0, 0], z[2, 0, 1] = float("nan"), 63.5
    q, s = R.quantize_per_token_head_ref(z, INT8_MODE)
    assert float(s[0, 0]) == float(np.float32(1e-6)) and torch.count_nonzero(q[0]) == 0
    assert float(s[1, 0]) == float(np.float32(1e-6))
    assert q[1, 0, :2].tolist() == [10, -4]
    assert float(s[2, 0]) == float(np.float32(63.5) / np.float32(127.0))
    assert q[2, 0, :2].tolist() == [-128, 127]


def test_per_token_int8_error_bound():
    g = torch.Generator().manual_seed(33)
    x = torch.randn(9, 8, 128, generator=g) * torch.rand(9, 8, 1, generator=g) * 50
    q, s = R.quantize_per_token_head_ref(x, INT8_MODE)
    deq = q.double() * s.double()[..., None]
    assert bool(((deq - x.double()).abs() <= s.double()[..., None] * (0.5 + 1e-5)).all())
    assert int(q.abs().amax()) == 127


@pytest.mark.parametrize("mode", [FP8_MODE, INT8_MODE])
def test_store_kvcache_quant_ref_matches_loop(mode):
    g = torch.Generator().manual_seed(34)
    T, H, D, N, bs = 11, 2, 16, 4, 4
    k = torch.randn(T, H, D, generator=g)
    v = torch.randn(T, H, D, generator=g)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::4] = -1
    cdt = torch.float8_e4m3fn if mode == FP8_MODE else torch.int8
    kc = torch.zeros(N, bs, H, D, dtype=cdt)
    vc = torch.zeros_like(kc)
    ks, vs = torch.ones(N, bs, H), torch.ones(N, bs, H)
    R.store_kvcache_quant_ref(k, v, kc, vc, ks, vs, slots, mode)
    for t in range(T):
        sl = int(slots[t])
        if sl == -1:
            continue
        for x, cache, sc in ((k, kc, ks), (v, vc, vs)):
            qrow, srow = R.quantize_per_token_head_ref(x[t:t + 1], mode)
            assert torch.equal(cache[sl // bs, sl % bs].view(torch.uint8), qrow[0].view(torch.uint8))
            assert torch.equal(sc[sl // bs, sl % bs], srow[0])
    untouched = torch.ones(N * bs, dtype=torch.bool)
    untouched[slots[slots >= 0]] = False
    assert bool((ks.view(-1, H)[untouched] == 1).all()) and bool((vs.view(-1, H)[untouched] == 1).all())
    assert torch.count_nonzero(kc.view(N * bs, -1)[untouched].view(torch.uint8)) == 0


def _tiny_token_quant(seed, mode, B=2, Hq=4, Hkv=2, D=16, N=12, bs=8, max_blocks=5):
    q, k, v, bt, ctx, _, _ = _tiny_decode(seed, B, Hq, Hkv, D, N, bs, max_blocks)
    k = k * torch.rand(N, bs, Hkv, 1, generator=torch.Generator().manual_seed(seed)) * 4
    kq, ks = R.quantize_per_token_head_ref(k.reshape(-1, Hkv, D), mode)
    vq, vs = R.quantize_per_token_head_ref(v.reshape(-1, Hkv, D), mode)
    return (q, kq.reshape(N, bs, Hkv, D), vq.reshape(N, bs, Hkv, D), ks.reshape(N, bs, Hkv),
            vs.reshape(N, bs, Hkv), bt, ctx)


@pytest.mark.parametrize("seed,mode", [(40, FP8_MODE), (41, INT8_MODE), (42, INT8_MODE)])
def test_decode_ref_per_token_matches_tile_literal(seed, mode):
    q, kq, vq, ks, vs, bt, ctx = _tiny_token_quant(seed, mode)
    got = R.paged_decode_ref(q, kq, vq, bt, ctx, 0.3, 4, 2, ks, vs)
    want = R.paged_decode_tile_literal(q, kq, vq, ks, vs, bt, ctx, 0.3, 4, 2)
    assert torch.allclose(got.double(), want, atol=1e-6, rtol=0)


def test_decode_ref_per_token_with_uniform_scales_is_per_tensor():
    # the same scale in every slot reduces to the per-tensor dequantisation
    q, kq, vq, ks, vs, bt, ctx = _tiny_token_quant(43, FP8_MODE)
    a = R.paged_decode_ref(q, kq, vq, bt, ctx, 0.3, 4, 2, torch.full_like(ks, 0.37),
                           torch.full_like(vs, 1.9))
    b = R.paged_decode_ref(q, kq, vq, bt, ctx, 0.3, 4, 2, 0.37, 1.9)
    assert torch.equal(a, b)
    # and per-token scales are per slot: scaling one slot's V scale moves the
    # output exactly as scaling that token's V values does
    b0, s0 = 0, int(bt[0, 0])
    vs2 = vs.clone()
    vs2[s0, 1] *= 3.0
    vdeq = vq.float() * vs[..., None]
    vdeq2 = vdeq.clone()
    vdeq2[s0, 1] *= 3.0
    kdeq = kq.float() * ks[..., None]
    got = R.paged_decode_ref(q, kq, vq, bt, ctx, 0.3, 4, 2, ks, vs2)
    want = R.paged_decode_ref(q, kdeq, vdeq2, bt, ctx, 0.3, 4, 2)
    assert torch.allclose(got, want, atol=1e-6)


def test_tile_literal_keeps_the_reference_hole_quirk():
    # a -1 block inside the context: the per-tensor kernels skip its tokens,
    # the reference's tile kernel adds exp(0 - m) per token to the denominator
    q, kq, vq, ks, vs, bt, ctx = _tiny_token_quant(44, INT8_MODE, max_blocks=5)
    ctx[:] = 5 * 8
    bt[0] = torch.arange(5, dtype=torch.int32)
    bt[1] = torch.arange(5, 10, dtype=torch.int32)
    bt[0, 2] = -1
    skip = R.paged_decode_ref(q, kq, vq, bt, ctx, 0.3, 4, 2, ks, vs)
    lit = R.paged_decode_tile_literal(q, kq, vq, ks, vs, bt, ctx, 0.3, 4, 2)
    assert torch.allclose(skip[1].double(), lit[1], atol=1e-6)
    assert not torch.allclose(skip[0].double(), lit[0], atol=1e-3)


# ---------------------------------------------------------------------------
# Decode-step metadata (model_runner.py:530-553, :621-640)
# ---------------------------------------------------------------------------
def test_decode_metadata_ref_matches_prepare_decode_except_at_block_ends():
    g = torch.Generator().manual_seed(50)
    bs = 16
    perm = torch.randperm(200, generator=g).tolist()
    for L in range(2, 120):
        nb = (L + bs - 1) // bs
        bt = perm[:nb]
        ctx, slots = R.decode_metadata_ref([bt], [L], bs)
        assert ctx == [L]
        literal = R.prepare_decode_slot_literal(bt, L, bs)
        if L % bs:
            assert slots == [literal]
        else:
            # the reference's formula lands on the last slot of block bt[-1] - 1
            assert literal == bt[-1] * bs - 1 and slots == [bt[-1] * bs + bs - 1]
        # the slot is where the prefill path would have written token L - 1
        assert slots[0] == bt[(L - 1) // bs] * bs + (L - 1) % bs


def test_decode_metadata_ref_padding_and_absent_blocks():
    ctx, slots = R.decode_metadata_ref([[3, 4], [7], [0, 0]], [20, 5, 0], 16)
    assert ctx == [20, 5, 0] and slots == [4 * 16 + 3, 7 * 16 + 4, -1]
    ctx, slots = R.decode_metadata_ref([[3, -1]], [20], 16)
    assert slots == [-1]


# ---------------------------------------------------------------------------
# Producer: RMSNorm + rotary embedding (layernorm.py:16-24,
# rotary_embedding.py:4-26, :100-109)
# ---------------------------------------------------------------------------
def _angles_cache(theta: torch.Tensor) -> torch.Tensor:
    """cos_sin rows for explicit angles (P, D/2) in float64."""
    return torch.cat([theta.cos(), theta.sin()], dim=-1)


def test_rope_ref_is_complex_rotation():
    g = torch.Generator().manual_seed(80)
    T, H, D = 9, 3, 16
    x = torch.randn(T, H, D, generator=g, dtype=torch.float64)
    theta = torch.rand(20, D // 2, generator=g, dtype=torch.float64) * 6.3
    pos = torch.randint(0, 20, (T,), generator=g)
    got = R.rope_ref(x, pos, _angles_cache(theta)).double()
    z = torch.complex(x[..., :D // 2], x[..., D // 2:]) * torch.exp(1j * theta[pos])[:, None, :]
    want = torch.cat([z.real, z.imag], dim=-1)
    assert torch.allclose(got, want, atol=1e-5)
    # position with zero angle is the identity; pair norms are preserved
    zero = _angles_cache(torch.zeros(1, D // 2, dtype=torch.float64))
    assert torch.allclose(R.rope_ref(x, torch.zeros(T, dtype=torch.int64), zero).double(), x, atol=1e-6)
    n_in = x[..., :D // 2] ** 2 + x[..., D // 2:] ** 2
    n_out = got[..., :D // 2] ** 2 + got[..., D // 2:] ** 2
    assert torch.allclose(n_in, n_out, atol=1e-4)


def test_rope_cache_composes_rotations():
    cs = R.rope_cos_sin_cache(10000.0, 32, 64).double()
    x = torch.randn(1, 2, 32, generator=torch.Generator().manual_seed(81), dtype=torch.float64)
    a, b = 17, 23
    ab = R.rope_ref(R.rope_ref(x, torch.tensor([a]), cs).double(), torch.tensor([b]), cs).double()
    direct = R.rope_ref(x, torch.tensor([a + b]), cs).double()
    assert torch.allclose(ab, direct, atol=2e-5)


def test_rms_norm_ref_invariants():
    g = torch.Generator().manual_seed(82)
    x = torch.randn(5, 4, 64, generator=g) * 7
    y = R.rms_norm_ref(x, torch.ones(64), 0.0).double()
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(5, 4, dtype=torch.float64), atol=1e-5)
    w = torch.rand(64, generator=g) + 0.5
    assert torch.allclose(R.rms_norm_ref(x, w, 0.0).double(), y * w.double(), atol=1e-5)
    c = torch.full((1, 1, 64), -3.0)
    assert torch.allclose(R.rms_norm_ref(c, w, 0.0), -w[None, None], atol=1e-6)
    # the result has x's dtype, rounded once
    xb = x.to(torch.bfloat16)
    assert R.rms_norm_ref(xb, w, 1e-5).dtype == torch.bfloat16


def test_qkv_norm_rope_ref_splits_columns():
    g = torch.Generator().manual_seed(83)
    Hq, Hkv, D, T = 4, 2, 16, 6
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g)
    cs = R.rope_cos_sin_cache(10000.0, D, 32)
    pos = torch.arange(T)
    q, k, v = R.qkv_norm_rope_ref(qkv, pos, Hq, Hkv, D, cs)
    assert torch.equal(v, qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D))
    assert torch.allclose(q, R.rope_ref(qkv[:, :Hq * D].reshape(T, Hq, D), pos, cs))
    assert torch.allclose(k, R.rope_ref(qkv[:, Hq * D:(Hq + Hkv) * D].reshape(T, Hkv, D), pos, cs))
