"""GPU tests of the engine slice (mkv.engine) on a 2-layer, small-vocabulary
copy of the Qwen3 shape (head_dim 128, 4 q / 2 kv heads), FP8 per-tensor KV,
block size 16, a token budget and a sequence cap that force chunked prefill,
queueing and mixed decode + prefill steps.

* The captured decode steps generate exactly the tokens of the same steps run
  eagerly (same kernels on the same bucket shapes).
* Step by step, the engine's logits match the same engine whose attention is
  the oracle's float64 restatement of the reference's attention
  (paged_prefill_ref / paged_decode_ref / flash_prefill_ref) on the same
  cache, with the sampled tokens forced equal so that both see the same
  inputs.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import announce
from mkv import context as C
from mkv import engine as E
from oracle import reference as R

pytestmark = pytest.mark.gpu

CFG = E.ModelConfig(vocab_size=512, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2,
                    head_dim=128, intermediate_size=512, max_position=4096)


def _prompts(seed, n=6):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(5, 101, (n,), generator=g).tolist()
    return [torch.randint(0, CFG.vocab_size, (L,), generator=g).tolist() for L in lens]


def _engine(dev, use_graphs=True, model_cls=E.Qwen3Model, kv="fp8_per_tensor", split=0):
    model = model_cls(CFG, dev, seed=5, block_size=16)
    return E.Engine(model, num_blocks=96, max_num_seqs=4, max_num_batched_tokens=64,
                    kv_cache_dtype=kv, max_model_len=256, seed=0, use_graphs=use_graphs,
                    decode_split_tokens=split)


@pytest.mark.parametrize("kv", ["fp8_per_tensor", "auto", "fp8_per_token_head", "int8_per_token_head"])
def test_captured_decode_generates_the_eager_tokens(dev, kv):
    announce(f"engine: captured vs eager decode, 2-layer model, {kv} KV")
    prompts = _prompts(11)
    outs = []
    for graphs in (True, False):
        eng = _engine(dev, graphs, kv=kv)
        outs.append(eng.generate(prompts, max_tokens=12))
        kinds = {s.kind for s in eng.stats}
        assert kinds == {"mixed", "decode"}, kinds
        assert all(len(o) == 12 for o in outs[-1])
        if kv == "fp8_per_tensor":
            assert all(float(s) != 1.0 for s in eng.model.scales()), "scales calibrated"
    assert outs[0] == outs[1]


class OracleAttentionModel(E.Qwen3Model):
    """The same model with the oracle's attention on the CPU in float64 over
    the layer's own (dequantised) cache, on every step (decode steps too:
    no fused producer + attention call)."""

    fuse_decode_step = False

    def attention(self, li, q, k, v):
        ctx = C.current_context()
        att = self.layers[li]["attn"]
        Hq, Hkv = self.cfg.num_heads, self.cfg.num_kv_heads
        sm = 1.0 / math.sqrt(self.cfg.head_dim)
        if att.kv_cache_dtype == "fp8_per_tensor":
            ks, vs = float(att.k_scale), float(att.v_scale)
        elif att.kv_cache_dtype == "auto":
            ks = vs = None
        else:  # per-token-head: the (N, bs, Hkv) scales the appends wrote
            ks, vs = att.k_scale.cpu(), att.v_scale.cpu()
        kc, vc = att.k_cache.cpu(), att.v_cache.cpu()
        if ctx.is_prefill and ctx.is_full_prefill:
            out = R.flash_prefill_ref(q.cpu().double(), k.cpu().double(), v.cpu().double(),
                                      ctx.cu_seqlens_q.cpu(), sm, Hq, Hkv)
        elif ctx.is_prefill:
            out = R.paged_prefill_ref(q.cpu().double(), kc, vc, ctx.block_tables.cpu(),
                                      ctx.context_lens.cpu(), ctx.cu_seqlens_q.cpu(),
                                      ctx.positions.cpu(), sm, Hq, Hkv, ks, vs)
        else:
            out = R.paged_decode_ref(q.cpu().double(), kc, vc, ctx.block_tables.cpu(),
                                     ctx.context_lens.cpu(), sm, Hq, Hkv, ks, vs)
        return out.to(q.dtype).to(q.device).reshape(q.shape[0], Hq * self.cfg.head_dim)


@pytest.mark.parametrize("split", [0, 32, -1])
def test_engine_logits_match_the_oracle_attention_engine(dev, monkeypatch, split):
    """Every step's logits against the same engine with the oracle's
    attention; decode by stream-K (split 0), by 32-token split-K and by the
    workgroup route (-1, one workgroup per sequence and KV head)."""
    announce(f"engine: logits vs the same engine with oracle attention, every step, split {split}")
    _logits_vs_oracle(dev, monkeypatch, split, "fp8_per_tensor")


@pytest.mark.parametrize("kv", ["fp8_per_token_head", "int8_per_token_head"])
def test_engine_per_token_head_kv_logits_match_the_oracle_attention_engine(dev, monkeypatch, kv):
    """The per-token-head KV modes through the engine (per-slot scales
    written by the producer's append; decode, chunked prefill and the mixed
    steps on the per-token-head kernels): every step's logits against the
    oracle-attention engine over its own codes and scales."""
    announce(f"engine: {kv} KV, logits vs the same engine with oracle attention, every step")
    _logits_vs_oracle(dev, monkeypatch, 0, kv)


def _logits_vs_oracle(dev, monkeypatch, split, kv):
    prompts = _prompts(12)
    eng = _engine(dev, True, split=split, kv=kv)
    ref = _engine(dev, False, model_cls=OracleAttentionModel, kv=kv)
    for e in (eng, ref):
        for p in prompts:
            e.add_request(p, max_tokens=6)
    forced = {}
    real_sample = E.sample

    def sample_forced(logits, temperature, gen):
        if "tok" in forced:
            return forced.pop("tok")
        return real_sample(logits, temperature, gen)

    monkeypatch.setattr(E, "sample", sample_forced)
    kinds = []
    worst = 0.0
    compared = 0
    for step in range(60):
        if eng.sched.done():
            break
        eng.step()
        kinds.append(eng.stats[-1].kind)
        sampled = eng.last_sampled
        if sampled:  # the reference engine samples exactly the engine's tokens
            forced["tok"] = torch.tensor(sampled, dtype=torch.int64, device=dev)
        ref.step()
        assert "tok" not in forced
        assert [r.tokens for r in eng.sched.running] == [r.tokens for r in ref.sched.running]
        if not sampled:
            continue
        got, want = eng.last_logits.float(), ref.last_logits.float()
        assert got.shape == want.shape == (len(sampled), CFG.vocab_size)
        err = float((got - want).abs().max())
        worst = max(worst, err)
        compared += 1
        assert err <= 3e-2, f"step {step} ({kinds[-1]}): max logit difference {err:.3e}"
    assert eng.sched.done() and ref.sched.done()
    assert "mixed" in kinds and "decode" in kinds and compared >= 6, kinds
    print(f"max logit difference over {compared} steps: {worst:.2e}")


# The end-to-end workload's model shape (Qwen3-0.6B: hidden 1024, 16 q / 8 kv
# heads, head_dim 128, intermediate 3072, vocab 151936) with 2 of its 28
# layers.
FULL = E.ModelConfig(num_layers=2)


def _full_engine(dev, model_cls, use_graphs, dtype, kv_cache_dtype="fp8_per_tensor"):
    model = model_cls(FULL, dev, dtype=dtype, seed=5, block_size=256)
    return E.Engine(model, num_blocks=40, max_num_seqs=8, max_num_batched_tokens=1024,
                    kv_cache_dtype=kv_cache_dtype, max_model_len=1024, seed=0, use_graphs=use_graphs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_engine_logits_full_shape_match_the_oracle_attention_engine(dev, monkeypatch, dtype):
    """The end-to-end workload's shape (Qwen3-0.6B attention and projections,
    vocab 151936, 256-token blocks, FP8 per-tensor KV, a 1024-token step
    budget with chunked prefill) on 2 layers and 8 prompts of 32-512 tokens:
    every step's logits (mixed prefill steps, then captured decode steps
    through the library's decode schedule) against the same engine with the
    oracle's float64 attention over its own cache.

    fp32 weights (the reference engine's default precision,
    model_runner.py:87): only the attention arithmetic differs, within 3e-2.
    bf16 weights (the end-to-end workload's): each attention output is one
    bf16 rounding of the oracle's or of the kernel's value, and a one-ulp
    difference there moves the hidden state by 2^-8 relative, which the
    layers after it carry to the logits; the bound is 6e-2 plus one bf16
    ulp of the logit (both engines round their logits to bf16), and the mean
    difference at most 1e-2."""
    announce(f"engine: full-shape (hidden 1024, 16/8 heads, vocab 151936, block 256), {dtype} weights, "
             "logits vs oracle attention")
    g = torch.Generator().manual_seed(55)
    lens = [int(x) for x in torch.randint(32, 513, (8,), generator=g)]
    lens[0], lens[1] = 512, 32
    prompts = [torch.randint(0, FULL.vocab_size, (L,), generator=g).tolist() for L in lens]
    eng = _full_engine(dev, E.Qwen3Model, True, dtype)
    ref = _full_engine(dev, OracleAttentionModel, False, dtype)
    for e in (eng, ref):
        for p in prompts:
            e.add_request(p, max_tokens=6)
    forced = {}
    real_sample = E.sample

    def sample_forced(logits, temperature, gen):
        if "tok" in forced:
            return forced.pop("tok")
        return real_sample(logits, temperature, gen)

    monkeypatch.setattr(E, "sample", sample_forced)
    kinds, worst, compared = [], 0.0, 0
    for step in range(40):
        if eng.sched.done():
            break
        eng.step()
        kinds.append(eng.stats[-1].kind)
        sampled = eng.last_sampled
        if sampled:
            forced["tok"] = torch.tensor(sampled, dtype=torch.int64, device=dev)
        ref.step()
        assert "tok" not in forced
        assert [r.tokens for r in eng.sched.running] == [r.tokens for r in ref.sched.running]
        if not sampled:
            continue
        got, want = eng.last_logits.float(), ref.last_logits.float()
        assert got.shape == want.shape == (len(sampled), FULL.vocab_size)
        diff = (got - want).abs()
        if dtype == torch.float32:
            tol = torch.full_like(want, 3e-2)
        else:
            tol = 6e-2 + torch.exp2(torch.floor(torch.log2(want.abs().clamp(min=2.0 ** -14))) - 7)
        err, mean = float(diff.max()), float(diff.mean())
        worst = max(worst, err)
        compared += 1
        print(f"step {step} ({kinds[-1]}, {len(sampled)} rows): max logit difference {err:.3e}, "
              f"mean {mean:.2e}, max |logit| {float(want.abs().max()):.2f}")
        assert bool((diff <= tol).all()), f"step {step} ({kinds[-1]}): max logit difference {err:.3e}"
        assert mean <= 1e-2, f"step {step} ({kinds[-1]}): mean logit difference {mean:.3e}"
    assert eng.sched.done() and ref.sched.done()
    assert kinds.count("mixed") >= 2 and kinds.count("decode") >= 4, kinds
    assert all(float(s) != 1.0 for s in eng.model.scales()), "scales calibrated"
    print(f"max logit difference over {compared} steps: {worst:.2e}; steps {kinds}")


class UnfusedModel(E.Qwen3Model):
    """The engine's model with each decode step's producer step and attention
    as two calls."""

    fuse_decode_step = False


@pytest.mark.parametrize("use_graphs,kv", [(True, "fp8_per_tensor"), (False, "fp8_per_tensor"), (True, "auto"),
                                           (True, "fp8_per_token_head"), (True, "int8_per_token_head")])
def test_fused_decode_steps_give_the_unfused_logits(dev, monkeypatch, use_graphs, kv):
    """The end-to-end workload's shape (2 layers, bf16 weights, FP8 per-tensor,
    bf16 or per-token-head KV, 8 prompts of 32-512 tokens): with each decode step's producer
    step and attention in one launch (mkv_qkv_norm_rope_append_decode),
    every step's logits are bit-identical to the two calls' and so are the
    generated tokens, captured or eager."""
    announce(f"engine: fused decode steps vs two calls, graphs {use_graphs}, kv {kv}")
    from mkv import _lib

    names = []
    real_call = _lib.call

    def spy(name, *args):
        names.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", spy)
    g = torch.Generator().manual_seed(56)
    lens = [int(x) for x in torch.randint(32, 513, (8,), generator=g)]
    prompts = [torch.randint(0, FULL.vocab_size, (L,), generator=g).tolist() for L in lens]
    eng = _full_engine(dev, E.Qwen3Model, use_graphs, torch.bfloat16, kv)
    ref = _full_engine(dev, UnfusedModel, use_graphs, torch.bfloat16, kv)
    for e in (eng, ref):
        for p in prompts:
            e.add_request(p, max_tokens=8)
    kinds, compared = [], 0
    for step in range(40):
        if eng.sched.done():
            break
        eng.step()
        ref.step()
        kinds.append(eng.stats[-1].kind)
        assert eng.last_sampled == ref.last_sampled, f"step {step}: tokens differ"
        if eng.last_sampled:
            assert torch.equal(eng.last_logits, ref.last_logits), f"step {step} ({kinds[-1]}): logits differ"
            compared += 1
    assert eng.sched.done() and ref.sched.done()
    assert "decode" in kinds and compared >= 6, kinds
    assert "mkv_qkv_norm_rope_append_decode" in names, "the fused call never ran"
