"""GPU parity of the fused greedy sampling + unmask step (fdllm_unmask_step) with the
torch statement of the reference rule (fast_v2_amd.e2e.sampler.greedy_with_confidence
+ threshold_unmask, i.e. modeling.py:2263-2270 and generation_functions.py:784-807).

Bar: tokens, unmask decisions, the stop rule and the counters exact; the confidence
within one ulp of the logits' type (the softmax sum is accumulated in another order
than torch's). The logits are drawn so that no confidence lies within an ulp of the
threshold and no two probabilities tie after rounding except where planted (an
exact tie between two equal logits, resolved to the first index).
"""
import pytest
import torch

from fast_v2_amd import ops
from fast_v2_amd.e2e import model as em
from fast_v2_amd.e2e import sampler as es

pytestmark = pytest.mark.gpu


def _torch_step(raw, x_sub, mask_id, thr, row_offset, finished, stop):
    L = x_sub.shape[1]
    logits = torch.cat([raw[:, :1], raw[:, :-1]], dim=1)[:, row_offset:row_offset + L]
    tok, conf = es.greedy_with_confidence(logits)
    masked = (x_sub == mask_id) & ~finished[:, None]
    unmask = es.threshold_unmask(tok, conf, masked, thr)
    new = torch.where(unmask, tok, x_sub)
    fin = finished | ((tok == stop) & unmask).any(dim=1) if stop is not None else finished.clone()
    left = ((new == mask_id) & ~finished[:, None] & ~fin[:, None]).sum()
    return tok, conf, new, fin, [int(unmask.sum()), int(left), int((new[:, 0] == mask_id).sum()), int(fin.sum())]


@pytest.mark.parametrize("V,R,L,row_offset", [(152064, 8, 8, 0), (152064, 32, 8, 8), (1000, 32, 8, 24), (4099, 9, 5, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_unmask_step_matches_torch(gpu, V, R, L, row_offset, dtype):
    g = torch.Generator().manual_seed(V + R + L + row_offset)
    B, mask_id, thr, stop = 6, V - 1, 0.9, 7
    raw = (torch.randn(B, R, V, generator=g) * 2).to(dtype)
    # peaked rows: confident positions (conf well above the threshold)
    for b in range(B):
        for r in range(R):
            if (b + r) % 3 == 0:
                raw[b, r, (b * 31 + r * 17) % (V - 1)] = 30.0
    raw[0, 0, 5] = raw[0, 0, 9] = 40.0   # an exact tie: the first index wins
    raw[2, 1, stop] = 50.0               # row 2 emits the stop token
    x_sub = torch.randint(0, V - 1, (B, L), generator=g)
    x_sub[torch.rand(B, L, generator=g) < 0.7] = mask_id
    x_sub[4] = mask_id
    finished = torch.zeros(B, dtype=torch.bool)
    finished[5] = True
    raw_g, x_g, fin_g = raw.to(gpu), x_sub.to(gpu), finished.to(gpu)
    print(f"case unmask V={V} R={R} L={L} off={row_offset} {dtype}", flush=True)
    tok, conf, new, fin, counts = _torch_step(raw_g, x_g.clone(), mask_id, thr, row_offset, fin_g.clone(), stop)
    sc = ops.unmask_step(raw_g, x_g, mask_id, thr, row_offset=row_offset, shift=1, finished=fin_g, stop_token=stop)
    assert torch.equal(sc.row_tok, tok)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    torch.testing.assert_close(sc.row_conf, conf.float(), atol=0, rtol=ulp)
    assert torch.equal(x_g, new)
    assert torch.equal(fin_g, fin)
    assert sc.counts.tolist() == counts


def test_fused_sampler_generation_matches_torch_rule(gpu):
    """The same HIP forwards with the fused step and with the torch rule give the same
    generation (2-layer model, batch 4, 96 new tokens)."""
    cfg = em.BlockDiffusionConfig(num_hidden_layers=2)
    model = em.build_model(cfg, gpu)
    x = torch.randint(0, cfg.vocab_size - 1, (4, 64), generator=torch.Generator().manual_seed(6)).to(gpu)
    a, st_a = es.generate(model, x, max_new_tokens=96, impl=es.HipStaticAttention(fused_sampler=True))
    b, st_b = es.generate(model, x, max_new_tokens=96, impl=es.HipStaticAttention(fused_sampler=False))
    print(f"forwards {st_a.forwards} vs {st_b.forwards}")
    assert torch.equal(a, b)
    assert st_a.step_tokens == st_b.step_tokens
