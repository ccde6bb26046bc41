"""Seeded synthetic inputs shaped like a Llama-3.1-8B attention layer (32 query
heads, 8 kv heads, head_dim 128, RoPE theta 500000).

Used by bench.py, tests and smoke() to build identical inputs on every run:
all tensors come from ``torch.Generator().manual_seed(seed)`` on the CPU in
fp32, then are cast to fp16 (and moved by the caller).

  K: no-RoPE keys z . diag(sigma) . W^T . s with W a random orthonormal
     1024x1024 (QR of a Gaussian), sigma_i = exp(-i/tau), tau = 384/ln(100)
     (the top 192 of 1024 components hold ~99% of the energy), s scales each
     dim to unit std; reshaped (8, 128) per token and RoPE'd at positions 0..T-1
     (rotate_half convention, theta = 500000).
  V: N(0, 1) with two outlier channels (flat indices randperm(1024)[:2]) x8.
  Q: N(0, 1) of shape (B, 32, 1, 128).
"""
import math

import torch

N_Q, N_KV, HD = 32, 8, 128
THETA = 500000.0


def inv_freq(hd: int = HD, theta: float = THETA) -> torch.Tensor:
    """1 / theta^(arange(0, hd, 2)/hd) in fp32 (the Llama default without scaling)."""
    return 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))


def apply_rope(x: torch.Tensor, positions: torch.Tensor, inv_f: torch.Tensor) -> torch.Tensor:
    """x (..., T, hd) fp32; rotate_half RoPE with fp32 phases fl(pos*theta)."""
    freqs = positions.float()[:, None] * inv_f[None, :].float()
    emb = torch.cat([freqs, freqs], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos + rot * sin


def make_kv(T: int, batch: int = 1, seed: int = 0, n_kv: int = N_KV, hd: int = HD):
    """Returns (k_rope fp16, v fp16) of shape (batch, n_kv, T, hd) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    D = n_kv * hd
    W, _ = torch.linalg.qr(torch.randn(D, D, generator=g))
    tau = 384.0 / math.log(100.0)
    sigma = torch.exp(-torch.arange(D, dtype=torch.float32) / tau)
    M = sigma[:, None] * W.T                       # rows scaled components
    s = 1.0 / M.pow(2).sum(0).sqrt()               # per-dim std -> 1
    z = torch.randn(batch * T, D, generator=g)
    kn = (z @ M) * s                               # (B*T, D) no-RoPE keys
    kn = kn.view(batch, T, n_kv, hd).permute(0, 2, 1, 3)
    k = apply_rope(kn, torch.arange(T), inv_freq(hd))
    v = torch.randn(batch * T, D, generator=g)
    outl = torch.randperm(D, generator=g)[:2]
    v[:, outl] *= 8.0
    v = v.view(batch, T, n_kv, hd).permute(0, 2, 1, 3)
    return k.half().contiguous(), v.half().contiguous()


def make_kv_device(T: int, batch: int, seed: int, device, n_kv: int = N_KV, hd: int = HD,
                   mix=None):
    """make_kv's distributions generated on the device (for the many-layer
    prefill benchmark): returns (k_rope fp16, v fp16, mix) with shapes
    (batch, n_kv, T, hd).  `mix` (the scaled component matrix, D x D) can be
    passed back in to skip its QR; it is built from ``seed`` on the CPU."""
    D = n_kv * hd
    if mix is None:
        g = torch.Generator().manual_seed(seed)
        W, _ = torch.linalg.qr(torch.randn(D, D, generator=g))
        tau = 384.0 / math.log(100.0)
        sigma = torch.exp(-torch.arange(D, dtype=torch.float32) / tau)
        M = sigma[:, None] * W.T
        mix = (M * (1.0 / M.pow(2).sum(0).sqrt())).to(device)
    gd = torch.Generator(device=device).manual_seed(seed + 7)
    z = torch.randn(batch * T, D, generator=gd, device=device)
    kn = (z @ mix).view(batch, T, n_kv, hd).permute(0, 2, 1, 3)
    k = apply_rope(kn, torch.arange(T, device=device), inv_freq(hd).to(device))
    v = torch.randn(batch * T, D, generator=gd, device=device)
    outl = torch.randperm(D, generator=gd, device=device)[:2]
    v[:, outl] *= 8.0
    v = v.view(batch, T, n_kv, hd).permute(0, 2, 1, 3)
    return k.half().contiguous(), v.half().contiguous(), mix


def make_q(batch: int = 1, seed: int = 0, n_q: int = N_Q, hd: int = HD):
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randn(batch, n_q, 1, hd, generator=g).half()


def make_stream_tokens(n: int, batch: int = 1, seed: int = 0, n_kv: int = N_KV, hd: int = HD):
    """n decode tokens of K/V ~ N(0,1) fp16, each (batch, n_kv, 1, hd)."""
    g = torch.Generator().manual_seed(seed + 2)
    k = torch.randn(n, batch, n_kv, 1, hd, generator=g).half()
    v = torch.randn(n, batch, n_kv, 1, hd, generator=g).half()
    return k, v


def random_orthonormal_basis(D: int = N_KV * HD, rank: int = 192, seed: int = 0):
    """Config-4 fixed PCA basis: first `rank` columns of the QR of a seeded Gaussian."""
    g = torch.Generator().manual_seed(seed + 3)
    W, _ = torch.linalg.qr(torch.randn(D, D, generator=g))
    return W[:, :rank].contiguous()
