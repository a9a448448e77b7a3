"""Argument guards of the drop-in wrappers and the kernels' own bounds:
shape errors raise before any launch, and a cu_seqlens_q whose last entry
exceeds the query rows (the wrappers cannot read it without a host sync)
makes the prefill kernel clamp each sequence's rows to the rows that exist
instead of reading or writing past q and out."""
from __future__ import annotations

import pytest
import torch

from conftest import announce, assert_close_out
import mkv
from mkv import attention as A
from mkv import workloads as W
from oracle import reference as R

pytestmark = pytest.mark.gpu


def test_flash_prefill_cu_seqlens_past_the_rows_is_clamped(dev):
    announce("flash prefill: cu_seqlens past the rows")
    g = torch.Generator().manual_seed(31)
    T, Hkv, G = 150, 2, 2
    q = torch.randn(T, Hkv * G, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 128, generator=g).to(torch.bfloat16)
    bad = torch.tensor([0, 40, T + 70], dtype=torch.int32)  # the last sequence claims 70 rows too many
    got = mkv.flash_attention_prefill(q.to(dev), k.to(dev), v.to(dev), bad.to(dev), 0.09,
                                      Hkv * G, Hkv, 128).cpu()
    want = R.flash_prefill_ref(q.double(), k.double(), v.double(), torch.tensor([0, 40, T]),
                               0.09, Hkv * G, Hkv)
    assert_close_out(got, want, got.dtype, 2e-3)


def test_paged_prefill_rejects_short_metadata(dev):
    announce("paged prefill: short cu_seqlens / block tables / positions")
    kc = torch.zeros(8, 16, 2, 128, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(6, 4, 128, dtype=torch.bfloat16, device=dev)
    bt = torch.zeros(3, 2, dtype=torch.int32, device=dev)
    cl = torch.tensor([2, 2, 2], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 2, 4, 6], dtype=torch.int32, device=dev)
    pos = torch.tensor([0, 1, 0, 1, 0, 1], device=dev)
    call = lambda **kw: A.paged_attention_prefill_triton(
        q, kc, kc, kw.get("bt", bt), cl, kw.get("cu", cu), kw.get("pos", pos), 0.1, 4, 2, 128, 16)
    call()  # consistent metadata runs
    with pytest.raises(ValueError):
        call(cu=cu[:3])
    with pytest.raises(ValueError):
        call(bt=bt[:2])
    with pytest.raises(ValueError):
        call(pos=pos[:5])


def test_decode_and_append_reject_bad_arguments(dev):
    announce("decode / append argument guards")
    kc = torch.zeros(8, 16, 2, 128, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(3, 4, 128, dtype=torch.bfloat16, device=dev)
    bt = torch.zeros(3, 2, dtype=torch.int32, device=dev)
    cl = torch.tensor([5, 9, 1], dtype=torch.int32, device=dev)
    A.paged_attention_decode(q, kc, kc, bt, cl, 0.1, 4, 2, 128, 16)
    with pytest.raises(ValueError):
        A.paged_attention_decode(q, kc, kc, bt[:2], cl, 0.1, 4, 2, 128, 16)
    with pytest.raises(ValueError):
        A.paged_attention_decode(q, kc, kc, bt, cl[:2], 0.1, 4, 2, 128, 16)
    x = torch.zeros(4, 2, 128, dtype=torch.bfloat16, device=dev)
    slots = torch.arange(4, device=dev)
    f8 = torch.zeros(8, 16, 2, 128, dtype=torch.float8_e4m3fn, device=dev)
    with pytest.raises(ValueError):
        A._append(x, x, f8, f8, slots)  # an fp8 cache without scales
    with pytest.raises((ValueError, AssertionError)):
        A.store_kvcache(x, x, kc, kc, slots[:3], 16)
