"""Model integration on the GPU: a tiny seeded Qwen2 (head_dim 128, 4 query / 2 kv
heads, 2 layers, fp32) generating through ``PagedPackedCache`` and the
``winnow_packed`` attention (the reference's test_packed_model.py:83-100 and
:359-371, which run on the CPU there).

* Packed pages: the HIP decode operator against the reconstruct path (dequantize
  the history on the GPU, then SDPA) on the same pool bytes: identical greedy
  tokens and logits within 1e-3 (test_packed_model.py:83-100 uses 1e-3), with the
  backend counters showing which operator served each step and no native SDPA.
* Dense pages (bf16): the HIP dense kernel against dense SDPA, and against HF's own
  generation with a DynamicCache on the bf16-rounded K/V, step by step.
* One decode step of a real layer against the float64 oracle (the operator-vs-fp64
  layer check of model_contract.py:158-221).

Prompts of different lengths are prefilled one at a time (the whole prompt as one
chunk), then decoded as one batch with explicit position ids, as the reference's
engine does (engine.py:183-195).
"""
from __future__ import annotations

import pytest
import torch

DEV = "cuda"
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    from tiny_qwen import tiny_qwen
    return tiny_qwen(DEV)


def _prompts(n, seed=1):
    from tiny_qwen import prompts
    return prompts(n, seed)


@torch.no_grad()
def _generate(model, prompts, max_new, *, backend, bit_width=4, dense_dtype=None, page_size=16, allow_tf32=False):
    from winnow_amd import packed_backend as pb
    cfg = model.config
    pool = pb.make_pool(cfg, bit_width=None if dense_dtype else bit_width, num_pages=96, page_size=page_size,
                        device=DEV, dense_dtype=dense_dtype)
    kq, vq = pb.quantizers_for(cfg, bit_width, DEV)
    D = pb.head_dim_of(cfg)
    model.config._attn_implementation = pb.ATTN_NAME
    owners = [f"r{i}" for i in range(len(prompts))]
    last = []
    for o, p in zip(owners, prompts):
        pool.ensure(o, len(p) + max_new)
        cache = pb.PagedPackedCache(pool, [o], [0], k_quant=kq, v_quant=vq, head_dim=D, decode_backend=backend,
                                    allow_tf32=allow_tf32)
        out = model(input_ids=torch.tensor([p], device=DEV), position_ids=torch.arange(len(p), device=DEV)[None],
                    past_key_values=cache, use_cache=True, logits_to_keep=1)
        last.append(out.logits[0, -1].float())
    toks = [[int(lg.argmax())] for lg in last]
    steps = [torch.stack(last)]
    lengths = [len(p) for p in prompts]
    for _ in range(max_new - 1):
        cache = pb.PagedPackedCache(pool, owners, lengths, k_quant=kq, v_quant=vq, head_dim=D,
                                    decode_backend=backend, allow_tf32=allow_tf32)
        ids = torch.tensor([[t[-1]] for t in toks], device=DEV)
        pos = torch.tensor([[L] for L in lengths], device=DEV)
        out = model(input_ids=ids, position_ids=pos, past_key_values=cache, use_cache=True, logits_to_keep=1)
        lengths = cache.lengths
        lg = out.logits[:, -1].float()
        steps.append(lg)
        for t, x in zip(toks, lg):
            t.append(int(x.argmax()))
    return toks, steps


@pytest.mark.parametrize("bw", [8, 4])
def test_packed_decode_matches_the_reconstruct_path(model, bw):
    """The first decode step reads the same prompt bytes in both runs: there the two
    operators agree to 1e-4 of the logit scale at 8 bits (the reconstruct side
    dequantizes with an error below 2^-16 per term, which large scores amplify).
    Every step also appends K/V computed from the previous layer's slightly
    different output, and a code can flip at a bucket boundary; the bar after that
    is the reference's 1e-3 of the logit scale at 8 bits (its test uses 8-bit codes)
    and 1e-2 at 4 bits, whose buckets are 16 times wider. Greedy tokens must not
    change. The operator alone is held to the float64 oracle below."""
    from winnow_amd import packed_backend as pb
    prompts = _prompts(3, seed=3)
    pb.BACKEND_COUNTS.clear()
    ref_toks, ref_steps = _generate(model, prompts, 12, backend="reconstruct_sdpa", bit_width=bw)
    assert pb.BACKEND_COUNTS["reconstruct_sdpa"] > 0
    pb.BACKEND_COUNTS.clear()
    toks, steps = _generate(model, prompts, 12, backend="auto", bit_width=bw)
    assert toks == ref_toks
    scale = max(1.0, max(x.abs().max().item() for x in ref_steps))
    first = (steps[1] - ref_steps[1]).abs().max().item()
    assert first < (1e-4 if bw == 8 else 1e-2) * scale, (first, scale)
    worst = max((a - b).abs().max().item() for a, b in zip(steps, ref_steps))
    assert worst < (1e-3 if bw == 8 else 1e-2) * scale, (worst, scale)
    assert pb.BACKEND_COUNTS["hip_packed"] == 11 * 2          # 11 decode steps x 2 layers
    assert pb.BACKEND_COUNTS["prefill_reconstruct_sdpa"] == 3 * 2
    assert pb.BACKEND_COUNTS["native_sdpa"] == 0


def test_allow_tf32_decode_keeps_the_greedy_tokens(model):
    """The cache's allow_tf32 reaches the operator (the TF32-class scan at 4 bits, n_rep
    2): the logits differ from the fp32-exact decode's, and greedy tokens equal the
    reconstruct path's. This random-weight model's q and k projections have norms near
    100, so its attention scores run to hundreds; TF32-class operands (11 significant
    bits) move such scores by tenths and the first decode step's logits by a few
    percent of their scale (the fp32-exact decode: 2e-5). The bar here is therefore
    1e-1 of the logit scale; the operator itself is held to the float64 decode of
    rounded operands at scores of that size (test_gpu_decode_tf32.py). The prompts'
    Q > 1 steps run the fused prefill over the packed pages, which allow_tf32 opens to
    fp32 queries (the same operand class)."""
    from winnow_amd import packed_backend as pb
    prompts = _prompts(3, seed=5)
    ref_toks, ref_steps = _generate(model, prompts, 10, backend="reconstruct_sdpa", bit_width=4)
    exact_toks, exact_steps = _generate(model, prompts, 10, backend="auto", bit_width=4)
    pb.BACKEND_COUNTS.clear()
    toks, steps = _generate(model, prompts, 10, backend="auto", bit_width=4, allow_tf32=True)
    assert pb.BACKEND_COUNTS["hip_packed"] == 9 * 2
    assert pb.BACKEND_COUNTS["prefill_hip_packed"] == 3 * 2
    assert toks == ref_toks == exact_toks
    assert not torch.equal(steps[1], exact_steps[1])
    scale = max(1.0, max(x.abs().max().item() for x in ref_steps))
    worst = max((a - b).abs().max().item() for a, b in zip(steps, ref_steps))
    assert worst < 1e-1 * scale, (worst, scale)


def test_dense_pages_hip_kernel_matches_dense_sdpa_and_native_generation(model):
    from transformers import DynamicCache
    from winnow_amd import packed_backend as pb
    prompts = _prompts(2, seed=5)
    pb.BACKEND_COUNTS.clear()
    toks, steps = _generate(model, prompts, 10, backend="auto", dense_dtype=torch.bfloat16)
    assert pb.BACKEND_COUNTS["hip_dense"] == 9 * 2
    ref_toks, ref_steps = _generate(model, prompts, 10, backend="dense_sdpa", dense_dtype=torch.bfloat16)
    assert toks == ref_toks
    # relative to the logit scale: an appended K/V value can round to the other bf16
    # neighbour when the previous layer's output differs in its last bits
    scale = max(1.0, max(x.abs().max().item() for x in ref_steps))
    worst = max((a - b).abs().max().item() for a, b in zip(steps, ref_steps))
    assert worst < 1e-3 * scale, (worst, scale)
    # HF's own generation, K/V rounded to bf16 as the pool stores them, one sequence at a time
    model.config._attn_implementation = "sdpa"

    class Bf16Cache(DynamicCache):
        def update(self, k, v, layer_idx, *a, **kw):
            return super().update(k.bfloat16().float(), v.bfloat16().float(), layer_idx, *a, **kw)

    with torch.no_grad():
        for i, p in enumerate(prompts):
            cache = Bf16Cache(config=model.config)
            ids = torch.tensor([p], device=DEV)
            native = []
            for _ in range(10):
                lg = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1).logits[0, -1]
                native.append(int(lg.float().argmax()))
                ids = torch.tensor([[native[-1]]], device=DEV)
            assert native == toks[i]


def test_one_layer_decode_step_against_the_float64_oracle(model):
    """Capture a real layer's decode query and packed cache handle, rerun the HIP
    operator on them and compare with the float64 reconstruct oracle."""
    from oracle import attention as oa
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    seen = []
    orig = pa.packed_decode_attention

    def spy(q, kv, scale, **kw):
        out = orig(q, kv, scale, **kw)
        seen.append((q.clone(), kv, scale, out.clone()))
        return out

    pa.packed_decode_attention = spy
    try:
        _generate(model, _prompts(2, seed=9), 3, backend="auto")
    finally:
        pa.packed_decode_attention = orig
    assert seen
    q, kv, scale, out = seen[-1]
    quant = lambda x: pa.Quantizer(x.Pi.cpu(), x.centroids.cpu(), x.bit_width)  # noqa: E731
    host = oa.OracleKV(kv.k_pages.cpu(), kv.k_norms.cpu(), kv.v_pages.cpu(), kv.v_norms.cpu(),
                       kv.page_table.cpu(), kv.seq_lens.cpu(), quant(kv.k_quant), quant(kv.v_quant), kv.head_dim)
    ref = oa.reconstruct_attention_f64(q.cpu().double(), host, scale)
    assert torch.allclose(out.cpu().double(), ref, atol=2e-3, rtol=1e-3), (out.cpu().double() - ref).abs().max()
