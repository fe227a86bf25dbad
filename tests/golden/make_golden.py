"""Write the golden vectors under tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py

The reference ships no golden vectors (its kernel tests draw inputs from seeds on
CUDA, cuda_bench/test_correctness.py:83-87), and nothing of the reference is
imported here. Expected outputs come from library routines on the CPU:

kv_decode_small.npz   block-decode attention, fp32, batch 1, 12 query / 2 KV heads,
                      head_dim 128, 512 cached prefix keys + a 32-token block, every
                      query sees all 544 keys, scale 1/sqrt(128); inputs ~ N(0,1)
                      from seed 0 (q, k, v in that order). `out` is
                      torch.nn.functional.scaled_dot_product_attention on the CPU
                      (fp32) after the GQA expand of tests/test_focus.py:216-219;
                      `out_f64` is the same product in float64 numpy.
gather_small.npz      gather + RMSNorm, bf16 hidden [2, 64, 256] (stored as the
                      exact fp32 values), int64 indices [2, 9] with repeats,
                      bf16 weight ~ N(1, 0.05), eps 1e-6; expected gathered rows
                      (numpy take) and normed rows in the Fast_dLLM_QwenRMSNorm
                      order computed with numpy float32 arithmetic and explicit
                      bf16 round-to-nearest-even.
"""
from pathlib import Path
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from fast_v2_amd import workloads  # noqa: E402  (input generator only)


def _bf16_round(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def kv_decode_small():
    wl = workloads.kv_decode_fp32_small(seed=0)
    q, k, v = wl.q, wl.k_cache, wl.v_cache
    B, Sq, H, D = q.shape
    Hkv = k.shape[2]
    qh = q.transpose(1, 2)
    kh = k.transpose(1, 2)[:, :, None].expand(-1, -1, H // Hkv, -1, -1).reshape(B, H, -1, D)
    vh = v.transpose(1, 2)[:, :, None].expand(-1, -1, H // Hkv, -1, -1).reshape(B, H, -1, D)
    out = F.scaled_dot_product_attention(qh, kh, vh, scale=wl.scale).transpose(1, 2).contiguous()
    q64, k64, v64 = (t.double().numpy() for t in (q, k, v))
    kx = np.repeat(k64, H // Hkv, axis=2)
    vx = np.repeat(v64, H // Hkv, axis=2)
    s = np.einsum("bqhd,bkhd->bhqk", q64, kx) * wl.scale
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    out64 = np.einsum("bhqk,bkhd->bqhd", p, vx)
    np.savez(HERE / "kv_decode_small.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(),
             seqlens=wl.seqlens.numpy(), scale=np.float64(wl.scale), out=out.numpy(),
             out_f64=out64)


def gather_small():
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn(2, 64, 256, generator=g).to(torch.bfloat16)
    hidden[0, 5] = 0.0
    idx = torch.randint(0, 64, (2, 9), generator=g)
    idx[0, 0] = 5
    w = (1 + 0.05 * torch.randn(256, generator=g)).to(torch.bfloat16)
    h = hidden.float().numpy()
    wf = w.float().numpy()
    gathered = np.stack([h[b, idx[b].numpy()] for b in range(2)])
    g32 = gathered.astype(np.float32)
    var = (g32 * g32).mean(axis=-1, dtype=np.float32, keepdims=True)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(1e-6))).astype(np.float32)
    pre = _bf16_round(g32 * inv)
    normed = _bf16_round(wf * pre)
    np.savez(HERE / "gather_small.npz", hidden=h, indices=idx.numpy(), weight=wf, eps=np.float64(1e-6),
             gathered=gathered, normed=normed)


if __name__ == "__main__":
    kv_decode_small()
    gather_small()
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))
