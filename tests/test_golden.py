"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still produces the committed outputs from the committed
inputs (a change to the oracle that alters any of them fails here).
GPU: the kernels reproduce them through the C ABI: the FP8 append byte for
byte (whole pools and scales), decode / prefill within 2e-3 (fp16 / bf16
KV) or 2e-2 (FP8 KV) plus half an output ulp.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import announce, assert_close_out
from mkv import attention as A
from oracle import reference as R

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name: str) -> dict:
    with np.load(GOLD / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def _f16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.float16)


def _fp8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.copy()).view(torch.float8_e4m3fn)


# ---------------------------------------------------------------------------
# CPU: the oracle reproduces the fixtures
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["a", "b"])
def test_oracle_reproduces_append_fixture(case):
    z = _load("append_fp8.npz")
    key, value = _bf16(z[f"{case}_key"]), _bf16(z[f"{case}_value"])
    N, bs = int(z["num_blocks"]), int(z["block_size"])
    kc = torch.zeros(N, bs, key.shape[1], key.shape[2], dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1) if case == "a" else torch.from_numpy(z["b_k_scale"].copy())
    vs = torch.ones(1) if case == "a" else torch.from_numpy(z["b_v_scale"].copy())
    R.store_kvcache_fp8_ref(key, value, kc, vc, ks, vs, torch.from_numpy(z["slots"]))
    assert np.array_equal(kc.view(torch.uint8).numpy(), z[f"{case}_k_cache"])
    assert np.array_equal(vc.view(torch.uint8).numpy(), z[f"{case}_v_cache"])
    assert np.array_equal(ks.numpy(), z[f"{case}_k_scale"])
    assert np.array_equal(vs.numpy(), z[f"{case}_v_scale"])


def _decode_inputs(kind: str):
    z = _load(f"decode_{kind}.npz")
    q = torch.from_numpy(z["q"])
    if kind == "f16":
        k, v, ks, vs = _f16(z["k_cache"]), _f16(z["v_cache"]), None, None
    else:
        k, v = _fp8(z["k_cache"]), _fp8(z["v_cache"])
        ks, vs = float(z["k_scale"]), float(z["v_scale"])
    return z, q, k, v, ks, vs


@pytest.mark.parametrize("kind", ["f16", "fp8"])
def test_oracle_reproduces_decode_fixture(kind):
    z, q, k, v, ks, vs = _decode_inputs(kind)
    got = R.paged_decode_ref(q, k, v, torch.from_numpy(z["block_tables"]),
                             torch.from_numpy(z["context_lens"]), float(z["scale"]),
                             int(z["num_heads"]), int(z["num_kv_heads"]), ks, vs)
    np.testing.assert_allclose(got.numpy(), z["expected"], rtol=0, atol=1e-6)


def _prefill_inputs():
    z = _load("prefill_bf16.npz")
    return (z, torch.from_numpy(z["q"]), _bf16(z["k_cache"]), _bf16(z["v_cache"]),
            torch.from_numpy(z["block_tables"]), torch.from_numpy(z["context_lens"]),
            torch.from_numpy(z["cu_seqlens_q"]), torch.from_numpy(z["positions"]))


def test_oracle_reproduces_prefill_fixture():
    z, q, k, v, bt, ctx, cu, pos = _prefill_inputs()
    got = R.paged_prefill_ref(q, k, v, bt, ctx, cu, pos, float(z["scale"]), int(z["num_heads"]),
                              int(z["num_kv_heads"]))
    np.testing.assert_allclose(got.numpy(), z["expected"], rtol=0, atol=1e-6)


# ---------------------------------------------------------------------------
# GPU: the kernels reproduce the fixtures
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("case", ["a", "b"])
def test_gpu_append_matches_fixture(dev, case):
    announce(f"golden append_fp8 case {case}")
    z = _load("append_fp8.npz")
    key, value = _bf16(z[f"{case}_key"]).to(dev), _bf16(z[f"{case}_value"]).to(dev)
    N, bs = int(z["num_blocks"]), int(z["block_size"])
    kc = torch.zeros(N, bs, key.shape[1], key.shape[2], dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, device=dev) if case == "a" else torch.from_numpy(z["b_k_scale"].copy()).to(dev)
    vs = torch.ones(1, device=dev) if case == "a" else torch.from_numpy(z["b_v_scale"].copy()).to(dev)
    A.store_kvcache_fp8(key, value, kc, vc, ks, vs, torch.from_numpy(z["slots"]).to(dev), bs,
                        "fp8_per_tensor")
    torch.cuda.synchronize()
    assert np.array_equal(kc.view(torch.uint8).cpu().numpy(), z[f"{case}_k_cache"])
    assert np.array_equal(vc.view(torch.uint8).cpu().numpy(), z[f"{case}_v_cache"])
    assert np.array_equal(ks.cpu().numpy(), z[f"{case}_k_scale"])
    assert np.array_equal(vs.cpu().numpy(), z[f"{case}_v_scale"])


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["f16", "fp8"])
def test_gpu_decode_matches_fixture(dev, kind):
    announce(f"golden decode {kind}")
    z, q, k, v, ks, vs = _decode_inputs(kind)
    Hq, Hkv = int(z["num_heads"]), int(z["num_kv_heads"])
    args = (q.to(dev), k.to(dev), v.to(dev))
    bt = torch.from_numpy(z["block_tables"]).to(dev)
    ctx = torch.from_numpy(z["context_lens"]).to(dev)
    if kind == "f16":
        got = A.paged_attention_decode(*args, bt, ctx, float(z["scale"]), Hq, Hkv, 128, k.shape[1])
    else:
        got = A.paged_attention_decode_quantized(*args, torch.tensor([ks], device=dev),
                                                 torch.tensor([vs], device=dev), bt, ctx,
                                                 float(z["scale"]), Hq, Hkv, 128, k.shape[1],
                                                 "fp8_per_tensor")
    want = torch.from_numpy(z["expected"])
    assert_close_out(got.cpu(), want, got.dtype, 2e-3 if kind == "f16" else 2e-2)


@pytest.mark.gpu
def test_gpu_prefill_matches_fixture(dev):
    announce("golden prefill bf16")
    z, q, k, v, bt, ctx, cu, pos = _prefill_inputs()
    got = A.paged_attention_prefill_triton(q.to(dev), k.to(dev), v.to(dev), bt.to(dev), ctx.to(dev),
                                           cu.to(dev), pos.to(dev), float(z["scale"]),
                                           int(z["num_heads"]), int(z["num_kv_heads"]), 128,
                                           k.shape[1])
    assert_close_out(got.cpu(), torch.from_numpy(z["expected"]), got.dtype, 2e-3)
