"""GPU parity of K1 (slot-mapped append, FP8 quantisation, calibration).

Bar: bit-exact.  Every byte of the pool is compared, including slots the
append must not touch.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from mkv import attention as A
from mkv import workloads as W
from oracle import fp8_codec
from oracle import reference as R

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def _u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


def test_append_fp8_workload_byte_identical(dev):
    announce("append fp8: 4096 tokens bf16 -> 1024x256x8x128 pool, 5% slot -1")
    w = W.append_fp8(seed=2)
    N, bs, H = w["num_blocks"], w["block_size"], w["num_kv_heads"]
    kc = torch.zeros(N, bs, H, 128, dtype=FP8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    A.store_kvcache_fp8(w["key"].to(dev), w["value"].to(dev), kc, vc, ks, vs,
                        w["slot_mapping"].to(dev), bs, "fp8_per_tensor")
    kr = torch.zeros(N, bs, H, 128, dtype=FP8)
    vr = torch.zeros_like(kr)
    ksr, vsr = torch.ones(1), torch.ones(1)
    R.store_kvcache_fp8_ref(w["key"], w["value"], kr, vr, ksr, vsr, w["slot_mapping"])
    assert float(ks) == float(ksr) and float(vs) == float(vsr)
    assert torch.equal(_u8(kc), kr.view(torch.uint8))
    assert torch.equal(_u8(vc), vr.view(torch.uint8))


@pytest.mark.parametrize("scale", [0.5, 1.0, 0.125, 0.0123, 7.3])
def test_fp8_encoding_exhaustive_bf16(dev, scale):
    announce(f"fp8 encode of all 65536 bf16 patterns, scale {scale}")
    bits = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16))
    x = bits.view(torch.bfloat16).reshape(64, 8, 128)
    slots = torch.arange(64, dtype=torch.int64)
    kc = torch.zeros(1, 64, 8, 128, dtype=FP8, device=dev)
    vc = torch.zeros_like(kc)
    s = torch.full((1,), scale, device=dev)
    A._append(x.to(dev), x.to(dev), kc, vc, slots.to(dev), s, s)
    got = _u8(kc).reshape(-1).numpy()
    want = R.fp8_quantize_ref(x, scale).view(torch.uint8).reshape(-1).numpy()
    xf = x.float().reshape(-1).numpy()
    nan = np.isnan(xf)
    bad = np.nonzero(got != want)[0]
    detail = [(hex(int(bits[i]) & 0xFFFF), hex(got[i]), hex(want[i])) for i in bad[:8]]
    assert np.array_equal(got[~nan], want[~nan]), detail
    # NaN inputs stay NaN (0x7f / 0xff) with the sign torch's CPU cast gives
    assert np.array_equal(got[nan] & 0x7F, np.full(int(nan.sum()), 0x7F, np.uint8)), detail
    assert np.array_equal(got, want), detail


def test_fp8_encoding_exhaustive_bf16_many_scales(dev):
    """All 65,536 bf16 patterns against torch's cast for 40 scales at once:
    log-uniform over 2^-40..2^40, powers of two, the calibration floor
    (bf16(1e-8) / 448), a subnormal fp32 scale and ratios near 448."""
    announce("fp8 encode of all 65536 bf16 patterns, 40 scales")
    g = torch.Generator().manual_seed(12)
    scales = torch.exp2(torch.rand(28, generator=g, dtype=torch.float64) * 80 - 40).float().tolist()
    scales += [2.0 ** -20, 2.0 ** 7, 1.0 / 448, 3.0, 1.0 / 3, 448.0 / 3, 0.1,
               float(torch.tensor(1e-8).to(torch.bfloat16).float() / 448), 1e-40, 6.5e4, 1.17e-38, 2.0 ** 60]
    bits = torch.from_numpy(np.arange(65536, dtype=np.uint16).view(np.int16))
    x = bits.view(torch.bfloat16).reshape(64, 8, 128)
    slots = torch.arange(64, dtype=torch.int64)
    xd = x.to(dev)
    for scale in scales:
        kc = torch.zeros(1, 64, 8, 128, dtype=FP8, device=dev)
        vc = torch.zeros_like(kc)
        s = torch.full((1,), scale, device=dev)
        A._append(xd, xd, kc, vc, slots.to(dev), s, s)
        got = _u8(kc).reshape(-1).numpy()
        want = R.fp8_quantize_ref(x, float(s)).view(torch.uint8).reshape(-1).numpy()
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (scale, [(hex(int(bits[i]) & 0xFFFF), hex(got[i]), hex(want[i])) for i in bad[:8]])


@pytest.mark.parametrize("scale", [0.37, 3.0e-3, 1.0 / 3])
def test_fp8_encoding_random_fp32_inputs(dev, scale):
    announce(f"fp8 encode of random fp32 inputs over 2^-20..2^12, scale {scale}")
    g = torch.Generator().manual_seed(11)
    T, H, D = 512, 8, 128
    mag = torch.exp2(torch.randint(-20, 12, (T, H, D), generator=g).float())
    x = torch.randn(T, H, D, generator=g) * mag
    slots = torch.randperm(T, generator=g).to(torch.int64)
    kc = torch.zeros(2, 256, H, D, dtype=FP8, device=dev)
    vc = torch.zeros_like(kc)
    s = torch.full((1,), scale, device=dev)
    A._append(x.to(dev), x.to(dev), kc, vc, slots.to(dev), s, s)
    want = torch.zeros(2 * 256, H, D, dtype=FP8)
    want[slots] = R.fp8_quantize_ref(x, float(s))
    assert torch.equal(_u8(kc).reshape(-1), want.view(torch.uint8).reshape(-1))
    # the independent codec agrees on the same bytes
    assert np.array_equal(_u8(kc).reshape(-1, H, D)[slots].reshape(-1).numpy(),
                          fp8_codec.quantize_per_tensor(x.reshape(-1).numpy(), float(s)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_copy_append_bit_exact_with_padding_and_bounds(dev, dtype):
    announce(f"copy append {dtype}")
    g = torch.Generator().manual_seed(5)
    T, H, D, N, bs = 300, 8, 128, 16, 32
    k = torch.randn(T, H, D, generator=g).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::7] = -1
    slots[5] = N * bs + 3  # outside the pool: must be skipped, not written
    slots[6] = -5
    kc = torch.full((N, bs, H, D), 7.0, dtype=dtype, device=dev)
    vc = torch.full((N, bs, H, D), 7.0, dtype=dtype, device=dev)
    A.store_kvcache(k.to(dev), v.to(dev), kc, vc, slots.to(dev), bs)
    kr = torch.full((N, bs, H, D), 7.0, dtype=dtype)
    vr = torch.full((N, bs, H, D), 7.0, dtype=dtype)
    keep = (slots >= 0) & (slots < N * bs)
    R.store_kvcache_ref(k[keep], v[keep], kr, vr, slots[keep])
    assert torch.equal(kc.cpu(), kr) and torch.equal(vc.cpu(), vr)


def test_append_from_strided_qkv_view(dev):
    announce("append from k/v views into a fused qkv buffer")
    g = torch.Generator().manual_seed(6)
    T, Hq, H, D, N, bs = 64, 32, 8, 128, 4, 256
    qkv = torch.randn(T, (Hq + 2 * H) * D, generator=g).to(torch.bfloat16).to(dev)
    k = qkv[:, Hq * D:(Hq + H) * D].view(T, H, D)
    v = qkv[:, (Hq + H) * D:].view(T, H, D)
    assert not v.is_contiguous()
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    kc = torch.zeros(N, bs, H, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    A.store_kvcache(k, v, kc, vc, slots.to(dev), bs)
    kr = torch.zeros(N, bs, H, D, dtype=torch.bfloat16)
    vr = torch.zeros_like(kr)
    R.store_kvcache_ref(k.cpu(), v.cpu(), kr, vr, slots)
    assert torch.equal(kc.cpu(), kr) and torch.equal(vc.cpu(), vr)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_device_calibration_matches_reference_rule(dev, dtype):
    announce(f"fp8 calibration {dtype}")
    g = torch.Generator().manual_seed(8)
    for mag in (1.0, 37.5, 1e-3, 900.0):
        k = (torch.randn(257, 8, 128, generator=g) * mag).to(dtype)
        v = (torch.randn(257, 8, 128, generator=g) * mag * 0.5).to(dtype)
        ks = torch.ones(1, device=dev)
        vs = torch.ones(1, device=dev)
        A.calibrate_fp8_per_tensor(k.to(dev), v.to(dev), ks, vs)
        assert float(ks) == R.calibrate_scale_ref(k), (dtype, mag)
        assert float(vs) == R.calibrate_scale_ref(v), (dtype, mag)
        # frozen: a second call with other data keeps the scales
        A.calibrate_fp8_per_tensor((k * 3).to(dev), (v * 3).to(dev), ks, vs)
        assert float(ks) == R.calibrate_scale_ref(k)


def test_calibration_sentinel_and_zero_input(dev):
    announce("fp8 calibration: sentinel 1.0 and all-zero input")
    # amax 448 -> scale 1.0, which is the sentinel: the next call calibrates again
    k = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    k[2, 1, 5] = 448.0
    v = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    A.calibrate_fp8_per_tensor(k.to(dev), v.to(dev), ks, vs)
    assert float(ks) == 1.0
    assert float(vs) == R.calibrate_scale_ref(v)
    k2 = k * 0.5
    A.calibrate_fp8_per_tensor(k2.to(dev), v.to(dev), ks, vs)
    assert float(ks) == R.calibrate_scale_ref(k2)
    # an fp16 zero input calibrates to 0 exactly as the reference does
    z = torch.zeros(3, 8, 128, dtype=torch.float16)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    A.calibrate_fp8_per_tensor(z.to(dev), z.to(dev), ks, vs)
    assert float(ks) == R.calibrate_scale_ref(z) == 0.0



@pytest.mark.parametrize("in_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_append_sentinel_fallback_calibrates_like_the_kernel(dev, in_dtype):
    """The append's own sentinel path (used after a scale tensor's first
    store_kvcache_fp8) gives the calibrate-once result: a scale reset to 1.0
    on an already-used tensor is calibrated from all rows (slot -1 included)
    and written back; a scale that is not 1.0 is left alone."""
    announce(f"fp8 append sentinel fallback, {in_dtype}")
    g = torch.Generator().manual_seed(71)
    T, H, N, bs = 96, 8, 16, 16
    key = (torch.randn(T, H, 128, generator=g) * 3).to(in_dtype)
    value = (torch.randn(T, H, 128, generator=g) * 0.5).to(in_dtype)
    key[5, 2, 9] = 40.0  # the amax sits in a padding row
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[5] = -1
    kc = torch.zeros(N, bs, H, 128, dtype=FP8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, device=dev)
    vs = torch.ones(1, device=dev)
    kd, vd, sd = key.to(dev), value.to(dev), slots.to(dev)
    A.store_kvcache_fp8(kd, vd, kc, vc, ks, vs, sd, bs, "fp8_per_tensor")  # calibrates
    assert ks._mkv_calibrated
    first = float(ks), float(vs)
    # reset only k_scale: the next call goes straight to the append kernel
    ks.fill_(1.0)
    kc.zero_()
    vc.zero_()
    A.store_kvcache_fp8(kd, vd, kc, vc, ks, vs, sd, bs, "fp8_per_tensor")
    kr = torch.zeros(N, bs, H, 128, dtype=FP8)
    vr = torch.zeros_like(kr)
    ksr, vsr = torch.ones(1), torch.tensor([first[1]])
    R.store_kvcache_fp8_ref(key, value, kr, vr, ksr, vsr, slots)
    assert float(ks) == float(ksr) == first[0]
    assert float(vs) == first[1]
    assert torch.equal(_u8(kc), kr.view(torch.uint8))
    assert torch.equal(_u8(vc), vr.view(torch.uint8))
    # every slot -1: nothing is written, but the sentinel is still calibrated
    ks.fill_(1.0)
    kc.zero_()
    A.store_kvcache_fp8(kd, vd, kc, vc, ks, vs, torch.full_like(sd, -1), bs, "fp8_per_tensor")
    assert float(ks) == first[0]
    assert torch.count_nonzero(_u8(kc)) == 0


@pytest.mark.parametrize("mode", ["fp8_per_tensor", "fp8_per_token_head", "copy"])
def test_append_key_and_value_of_different_dtypes(dev, mode):
    """Regression: an fp32 key (a rotated k promoted by an fp32 cos/sin table)
    next to a bf16 value.  Both are widened to fp32 before the ABI call (it
    reads both with one dtype); the per-tensor scales are calibrated each in
    its own tensor's dtype, as the reference does."""
    announce(f"append, fp32 key + bf16 value, {mode}")
    g = torch.Generator().manual_seed(73)
    T, H, N, bs = 80, 8, 12, 16
    key = torch.randn(T, H, 128, generator=g) * 3
    value = (torch.randn(T, H, 128, generator=g) * 0.7).to(torch.bfloat16)
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[::6] = -1
    kd, vd, sd = key.to(dev), value.to(dev), slots.to(dev)
    if mode == "copy":
        kc = torch.zeros(N, bs, H, 128, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        A.store_kvcache(kd, vd, kc, vc, sd, bs)
        kr, vr = torch.zeros(N, bs, H, 128, dtype=torch.bfloat16), torch.zeros(N, bs, H, 128, dtype=torch.bfloat16)
        R.store_kvcache_ref(key, value, kr, vr, slots)
        assert torch.equal(kc.cpu().view(torch.int16), kr.view(torch.int16))
        assert torch.equal(vc.cpu().view(torch.int16), vr.view(torch.int16))
        return
    kc = torch.zeros(N, bs, H, 128, dtype=FP8, device=dev)
    vc = torch.zeros_like(kc)
    if mode == "fp8_per_tensor":
        ks, vs = torch.ones(1, device=dev), torch.ones(1, device=dev)
        for _ in range(2):  # the second call takes the calibrated path
            A.store_kvcache_fp8(kd, vd, kc, vc, ks, vs, sd, bs, mode)
        kr, vr = torch.zeros(N, bs, H, 128, dtype=FP8), torch.zeros(N, bs, H, 128, dtype=FP8)
        ksr, vsr = torch.ones(1), torch.ones(1)
        R.store_kvcache_fp8_ref(key, value, kr, vr, ksr, vsr, slots)
        assert float(ks) == float(ksr) and float(vs) == float(vsr)
    else:
        ks = torch.ones(N, bs, H, device=dev)
        vs = torch.ones_like(ks)
        A.store_kvcache_fp8(kd, vd, kc, vc, ks, vs, sd, bs, mode)
        kr, vr = torch.zeros(N, bs, H, 128, dtype=FP8), torch.zeros(N, bs, H, 128, dtype=FP8)
        ksr, vsr = torch.ones(N, bs, H), torch.ones(N, bs, H)
        R.store_kvcache_quant_ref(key, value.float(), kr, vr, ksr, vsr, slots, mode)
        assert torch.equal(ks.cpu(), ksr) and torch.equal(vs.cpu(), vsr)
    assert torch.equal(_u8(kc), kr.view(torch.uint8))
    assert torch.equal(_u8(vc), vr.view(torch.uint8))
