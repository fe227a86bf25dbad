"""Pins the gather + RMSNorm oracle (CPU only, no GPU, no HIP library).

Checks: the committed golden vectors (numpy take + float32 RMSNorm in the
Fast_dLLM_QwenRMSNorm rounding order, modeling.py:427-432), closed forms
(zero row -> 0, constant row c -> c / sqrt(c^2 + eps), unit RMS), agreement of
the torch and float64 numpy restatements in all three weight modes, the
bf16 round-to-nearest-even helper against torch's own conversion, and planted
mistakes (weight applied before the bf16 rounding; a missing eps; a wrong
gather axis) that must fail the golden check.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import gather_rmsnorm as og

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden():
    z = np.load(GOLDEN / "gather_small.npz")
    return {k: z[k] for k in z.files}


def _bf16_ulps(a, b) -> int:
    ai = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).int()
    bi = torch.from_numpy(np.ascontiguousarray(b, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).int()
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return int((ai - bi).abs().max())


def test_golden_torch_restatement():
    z = _golden()
    hidden = torch.from_numpy(z["hidden"]).to(torch.bfloat16)
    assert torch.equal(hidden.float(), torch.from_numpy(z["hidden"]))  # stored values are exact bf16
    idx = torch.from_numpy(z["indices"])
    w = torch.from_numpy(z["weight"]).to(torch.bfloat16)
    g, n = og.ref_gather_input_rmsnorm(hidden, idx, w, float(z["eps"]))
    assert torch.equal(g.float(), torch.from_numpy(z["gathered"]))
    # fp32 summation order may move the pre-weight value to a neighbouring bf16
    assert _bf16_ulps(n.float().numpy(), z["normed"]) <= 1
    assert (n.float().numpy() == z["normed"]).mean() > 0.99


def test_golden_numpy_restatement():
    z = _golden()
    g, n = og.gather_rmsnorm_np(z["hidden"], z["indices"], z["weight"], float(z["eps"]),
                                og.NORM_WEIGHT_AFTER_CAST, "bf16")
    np.testing.assert_array_equal(g, z["gathered"])
    assert _bf16_ulps(n, z["normed"]) <= 1
    assert (n == z["normed"]).mean() > 0.99


def test_golden_zero_row_gives_zero():
    z = _golden()
    # the fixture plants hidden[0, 5] = 0 and indices[0, 0] = 5
    assert z["indices"][0, 0] == 5 and not z["hidden"][0, 5].any()
    assert not z["normed"][0, 0].any()


def test_planted_weight_before_rounding_fails_golden():
    """Applying the weight in fp32 before the bf16 rounding (the .cu kernel order)
    is a different function: it must not reproduce the model-path golden."""
    z = _golden()
    _, n = og.gather_rmsnorm_np(z["hidden"], z["indices"], z["weight"], float(z["eps"]),
                                og.NORM_WEIGHT_FP32, "bf16")
    assert (n != z["normed"]).mean() > 0.05


def test_planted_missing_eps_and_wrong_axis_fail_golden():
    z = _golden()
    h = z["hidden"].astype(np.float64)
    idx = z["indices"]
    g = np.stack([h[b, idx[b]] for b in range(h.shape[0])])
    with np.errstate(invalid="ignore", divide="ignore"):
        no_eps = og.round_to(z["weight"] * og.round_to(g / np.sqrt((g * g).mean(-1, keepdims=True)), "bf16"),
                             "bf16")
    # the zero row turns into NaN without eps
    assert np.isnan(no_eps).any()
    wrong_axis = np.stack([h[idx[b] % h.shape[0], :, :][:, 0] for b in range(h.shape[0])])
    assert not np.array_equal(wrong_axis, z["gathered"])


@pytest.mark.parametrize("mode", [og.NORM_PLAIN, og.NORM_WEIGHT_FP32, og.NORM_WEIGHT_AFTER_CAST])
def test_torch_and_numpy_restatements_agree(mode):
    g = torch.Generator().manual_seed(mode)
    hidden = (2 * torch.randn(2, 40, 384, generator=g)).to(torch.bfloat16)
    idx = torch.randint(0, 40, (2, 11), generator=g)
    w = (1 + 0.05 * torch.randn(384, generator=g)).to(torch.bfloat16)
    if mode == og.NORM_PLAIN:
        tg, tn = og.ref_gather_pair_plain(hidden, idx, 1e-6)
    elif mode == og.NORM_WEIGHT_FP32:
        tn = og.ref_gather_rmsnorm_fp32w(hidden, idx, w, 1e-6)
        tg = torch.stack([hidden[b, idx[b]] for b in range(2)])
    else:
        tg, tn = og.ref_gather_input_rmsnorm(hidden, idx, w, 1e-6)
    ng, nn = og.gather_rmsnorm_np(hidden.float().numpy(), idx.numpy(), w.float().numpy(), 1e-6, mode, "bf16")
    np.testing.assert_array_equal(tg.float().numpy(), ng)
    assert _bf16_ulps(tn.float().numpy(), nn) <= (2 if mode == og.NORM_WEIGHT_AFTER_CAST else 1)


def test_closed_forms():
    H = 512
    hidden = np.zeros((1, 3, H), dtype=np.float32)
    hidden[0, 1] = 0.75
    hidden[0, 2] = og.round_to(np.linspace(-4, 4, H), "bf16")
    w = np.ones(H, dtype=np.float32)
    _, n = og.gather_rmsnorm_np(hidden, np.array([[0, 1, 2]]), w, 1e-6, og.NORM_WEIGHT_AFTER_CAST, "bf16")
    assert not n[0, 0].any()
    np.testing.assert_allclose(n[0, 1], 0.75 / np.sqrt(0.75 ** 2 + 1e-6), rtol=4e-3)
    assert abs(np.sqrt((n[0, 2].astype(np.float64) ** 2).mean()) - 1.0) < 5e-3


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(100000, generator=g) * torch.exp(4 * torch.randn(100000, generator=g))
    # exact ties: values halfway between two bf16 numbers
    ties = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(2.0 + 2 ** -7), 3.0 + 2 ** -7], dtype=torch.float32)
    x = torch.cat([x, ties])
    exp = x.to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(og.round_f32_to_bf16(x.numpy()), exp)


def test_scatter_oracle_against_torch_scatter_and_round_trip():
    """scatter_rows_np (fused_gather_norm.cu:79-119) against torch's scatter_ into both
    destinations; gathering the scattered rows back gives the values; rows no index names
    keep their old contents; an out-of-range index changes nothing; a planted off-by-one
    row index fails."""
    g = torch.Generator().manual_seed(3)
    B, S, T, H = 3, 50, 11, 24
    vals = torch.randn(B, T, H, generator=g)
    idx = torch.stack([torch.randperm(S, generator=g)[:T] for _ in range(B)])
    cache = torch.randn(B, S, H, generator=g)
    cur = torch.randn(B, S, H, generator=g)
    c, u = og.scatter_rows_np(vals.numpy(), idx.numpy(), cache.numpy(), cur.numpy())
    ii = idx.unsqueeze(-1).expand(-1, -1, H)
    np.testing.assert_array_equal(c, cache.clone().scatter_(1, ii, vals).numpy())
    np.testing.assert_array_equal(u, cur.clone().scatter_(1, ii, vals).numpy())
    for b in range(B):
        np.testing.assert_array_equal(c[b, idx[b].numpy()], vals[b].numpy())
        untouched = np.setdiff1d(np.arange(S), idx[b].numpy())
        np.testing.assert_array_equal(c[b, untouched], cache[b, untouched].numpy())
        np.testing.assert_array_equal(u[b, untouched], cur[b, untouched].numpy())
    bad = idx.clone()
    bad[1, 4] = S
    bad[2, 0] = -1
    c2, u2 = og.scatter_rows_np(vals.numpy(), bad.numpy(), cache.numpy(), None)
    assert u2 is None
    np.testing.assert_array_equal(c2[1, idx[1, 4]], cache[1, idx[1, 4]].numpy())
    np.testing.assert_array_equal(c2[2, idx[2, 0]], cache[2, idx[2, 0]].numpy())
    planted, _ = og.scatter_rows_np(vals.numpy(), ((idx + 1) % S).numpy(), cache.numpy())
    assert not np.array_equal(planted, c)
