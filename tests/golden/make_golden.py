"""Write the golden fixtures used by tests/test_golden.py.

Small seeded inputs and the oracle's outputs (oracle/reference.py, itself
pinned by tests/test_oracle.py) for:

* append_fp8.npz      per-tensor FP8 append: (A) calibrate-once from the 1.0
                      sentinel over all rows including slot -1 rows, (B) a
                      fixed scale with NaN, +-inf, saturating, tiny and -0.0
                      inputs; whole K/V pools as bytes.
* decode_f16.npz      paged decode, fp16 KV, fp32 q, GQA 4, holes (-1) and
                      padding in the block tables, context 1 / 37 / 70.
* decode_fp8.npz      the same with FP8 e4m3fn KV and per-tensor scales.
* prefill_bf16.npz    chunked prefill over the paged cache, bf16 KV, fp32 q.

The reference's own kernels are Triton and need an NVIDIA GPU, and its
repository holds no golden vectors for this path, so these vectors come from
the oracle.  Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import reference as R  # noqa: E402


def _u8(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy()


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _tables(ctx, bs, N, g, holes=()):
    mb = max((int(c) + bs - 1) // bs for c in ctx) + 1  # one padding column
    bt = torch.full((len(ctx), mb), -1, dtype=torch.int32)
    perm = torch.randperm(N, generator=g).tolist()
    for b, c in enumerate(ctx):
        for j in range((int(c) + bs - 1) // bs):
            bt[b, j] = perm.pop()
    for b, j in holes:
        bt[b, j] = -1
    return bt


def append_fp8():
    g = torch.Generator().manual_seed(101)
    N, bs, H, D, T = 4, 16, 2, 128, 40
    slots = torch.randperm(N * bs, generator=g)[:T].to(torch.int64)
    slots[[3, 17, 29]] = -1
    out = {"slots": slots.numpy(), "num_blocks": N, "block_size": bs}
    # (A) calibration from the sentinel; the largest |x| sits in a slot -1 row
    key = (torch.randn(T, H, D, generator=g) * 3).to(torch.bfloat16)
    value = (torch.randn(T, H, D, generator=g) * 0.5).to(torch.bfloat16)
    key[17, 1, 5] = -41.0
    kc = torch.zeros(N, bs, H, D, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ks, vs = torch.ones(1), torch.ones(1)
    R.store_kvcache_fp8_ref(key, value, kc, vc, ks, vs, slots)
    out.update(a_key=_u16(key), a_value=_u16(value), a_k_cache=_u8(kc), a_v_cache=_u8(vc),
               a_k_scale=ks.numpy(), a_v_scale=vs.numpy())
    # (B) fixed scale, special values
    key = (torch.randn(T, H, D, generator=g) * 10).to(torch.bfloat16)
    value = (torch.randn(T, H, D, generator=g) * 10).to(torch.bfloat16)
    specials = [float("nan"), -float("nan"), float("inf"), -float("inf"), 1e4, -1e4, 1e-6, -1e-6,
                -0.0, 0.0, 22.4, -22.4]
    for i, x in enumerate(specials):
        key[i, 0, i] = x
        value[i, 1, 2 * i] = x
    kc = torch.zeros(N, bs, H, D, dtype=torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    ks, vs = torch.tensor([0.05]), torch.tensor([0.03125])
    R.store_kvcache_fp8_ref(key, value, kc, vc, ks, vs, slots)
    out.update(b_key=_u16(key), b_value=_u16(value), b_k_cache=_u8(kc), b_v_cache=_u8(vc),
               b_k_scale=ks.numpy(), b_v_scale=vs.numpy())
    np.savez_compressed(HERE / "append_fp8.npz", **out)


def decode(kind: str):
    g = torch.Generator().manual_seed(102 if kind == "f16" else 103)
    B, Hq, Hkv, D, bs, N = 3, 8, 2, 128, 16, 10
    ctx = torch.tensor([1, 37, 70], dtype=torch.int64)
    bt = _tables(ctx, bs, N, g, holes=[(2, 2)])
    q = torch.randn(B, Hq, D, generator=g)
    k = torch.randn(N, bs, Hkv, D, generator=g)
    v = torch.randn(N, bs, Hkv, D, generator=g)
    scale = 1.0 / 128 ** 0.5
    out = dict(q=q.numpy(), block_tables=bt.numpy(), context_lens=ctx.numpy(), scale=np.float32(scale),
               num_heads=Hq, num_kv_heads=Hkv)
    if kind == "f16":
        k, v = k.half(), v.half()
        exp = R.paged_decode_ref(q, k, v, bt, ctx, scale, Hq, Hkv)
        out.update(k_cache=_u16(k), v_cache=_u16(v))
    else:
        kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
        ks, vs = R.calibrate_scale_ref(kb), R.calibrate_scale_ref(vb)
        k, v = R.fp8_quantize_ref(kb, ks), R.fp8_quantize_ref(vb, vs)
        exp = R.paged_decode_ref(q, k, v, bt, ctx, scale, Hq, Hkv, ks, vs)
        out.update(k_cache=_u8(k), v_cache=_u8(v), k_scale=np.float32(ks), v_scale=np.float32(vs))
    out["expected"] = exp.numpy()
    np.savez_compressed(HERE / f"decode_{kind}.npz", **out)


def prefill_bf16():
    g = torch.Generator().manual_seed(104)
    Hq, Hkv, D, bs, N = 4, 2, 128, 16, 6
    prior, qlen = [20, 0], [5, 9]
    ctx = torch.tensor([p + n for p, n in zip(prior, qlen)], dtype=torch.int64)
    bt = _tables(ctx, bs, N, g)
    cu = torch.tensor([0, qlen[0], qlen[0] + qlen[1]], dtype=torch.int32)
    pos = torch.tensor([p + j for p, n in zip(prior, qlen) for j in range(n)], dtype=torch.int64)
    q = torch.randn(int(cu[-1]), Hq, D, generator=g)
    k = torch.randn(N, bs, Hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(N, bs, Hkv, D, generator=g).to(torch.bfloat16)
    scale = 1.0 / 128 ** 0.5
    exp = R.paged_prefill_ref(q, k, v, bt, ctx, cu, pos, scale, Hq, Hkv)
    np.savez_compressed(HERE / "prefill_bf16.npz", q=q.numpy(), k_cache=_u16(k), v_cache=_u16(v),
                        block_tables=bt.numpy(), context_lens=ctx.numpy(), cu_seqlens_q=cu.numpy(),
                        positions=pos.numpy(), scale=np.float32(scale), num_heads=Hq,
                        num_kv_heads=Hkv, expected=exp.numpy())


if __name__ == "__main__":
    append_fp8()
    decode("f16")
    decode("fp8")
    prefill_bf16()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
