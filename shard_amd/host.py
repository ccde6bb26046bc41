"""Host-side (CPU, tiny) pieces of the compressed-KV path.

These run once per layer or once per process and produce small tables that
the kernels consume: the DP bit allocation of the PCA components, the
Lloyd-Max codebook of the decode stream, the stream sign vector, and the
model's RoPE inverse frequencies.
"""
import math

import torch

# ---------------------------------------------------------------------------
# DP bit allocation (rope.py:49-84)
# ---------------------------------------------------------------------------
_GROUP, _OPTIONS, _DROP, _UNIT = 64, (0, 2, 4, 6, 8), 4.0, 16


def dp_bit_allocation(variances, total_budget):
    """Bits per component: groups of 64 components get 0/2/4/6/8 bits so the
    total cost (ceil(64*bits/16) units per group, <= budget//16 + 1 units)
    minimizes sum of err, err = 4*var for a dropped group, var/(3*4^bits)
    otherwise.  Ties keep the first option / the smallest budget index
    (rope.py:49-84)."""
    v = [float(x) for x in torch.as_tensor(variances).float().cpu().tolist()]
    d = len(v)
    ng = (d + _GROUP - 1) // _GROUP
    sizes = [min(_GROUP, d - g * _GROUP) for g in range(ng)]
    # group sums in fp32 order of torch.sum over the slice
    gv = [torch.tensor(v[g * _GROUP: g * _GROUP + sizes[g]], dtype=torch.float32).sum().item()
          for g in range(ng)]
    units = total_budget // _UNIT + 1
    inf = float("inf")
    cost_tab = [[0 if b == 0 else (sizes[g] * b + _UNIT - 1) // _UNIT for b in _OPTIONS]
                for g in range(ng)]
    best = [[inf] * (units + 1) for _ in range(ng + 1)]
    choice = [[0] * (units + 1) for _ in range(ng + 1)]
    best[0] = [0.0] * (units + 1)
    for g in range(ng):
        for u in range(units + 1):
            for oi, bits in enumerate(_OPTIONS):
                c = cost_tab[g][oi]
                if u - c < 0:
                    continue
                err = gv[g] * _DROP if bits == 0 else gv[g] / (3.0 * (1 << (2 * bits)))
                val = best[g][u - c] + err
                if val < best[g + 1][u]:
                    best[g + 1][u] = val
                    choice[g + 1][u] = bits
    u = min(range(units + 1), key=lambda i: best[ng][i])
    alloc = [0] * d
    for g in range(ng - 1, -1, -1):
        bits = choice[g + 1][u]
        alloc[g * _GROUP: g * _GROUP + sizes[g]] = [bits] * sizes[g]
        if bits > 0:
            u -= (sizes[g] * bits + _UNIT - 1) // _UNIT
    return alloc


# ---------------------------------------------------------------------------
# Lloyd-Max codebook of the decode stream (streaming.py:11-57)
# ---------------------------------------------------------------------------
# Acklam's rational approximation of the normal quantile (published constants).
_ACK_A = (-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
          1.383577518672690e+02, -3.066479806614716e+01, 2.506628277459239e+00)
_ACK_B = (-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
          6.680131188771972e+01, -1.328068155288572e+01)
_ACK_C = (-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
          -2.549732539343734e+00, 4.374664141464968e+00, 2.938163982698783e+00)
_ACK_D = (7.784695709041462e-03, 3.224671290700398e-01, 2.445134137142996e+00,
          3.754408661907416e+00)


def _poly(cs, x):
    acc = cs[0]
    for c in cs[1:]:
        acc = acc * x + c
    return acc


def normal_quantile(p: float) -> float:
    """Acklam's approximation, same evaluation order as streaming.py:20-33."""
    lo = 0.02425
    if p < lo:
        q = math.sqrt(-2 * math.log(p))
        return _poly(_ACK_C, q) / (_poly(_ACK_D, q) * q + 1)
    if p <= 1 - lo:
        q = p - 0.5
        r = q * q
        return _poly(_ACK_A, r) * q / (_poly(_ACK_B, r) * r + 1)
    q = math.sqrt(-2 * math.log(1 - p))
    return -_poly(_ACK_C, q) / (_poly(_ACK_D, q) * q + 1)


_codebooks = {}


def lloyd_max_codebook(d: int, bits: int, n_iter: int = 100) -> torch.Tensor:
    """Lloyd-Max levels for N(0, 1/d) (streaming.py:35-51): quantile seeds, then
    up to n_iter centroid-condition updates in double precision; an update whose
    largest step is < 1e-9 ends the loop without being taken.  fp32 result."""
    key = (d, bits, n_iter)
    if key in _codebooks:
        return _codebooks[key]
    n = 1 << bits
    sigma = 1.0 / math.sqrt(d)
    c = [normal_quantile((i + 0.5) / n) * sigma for i in range(n)]
    s2pi = math.sqrt(2 * math.pi)
    s2 = math.sqrt(2)
    for _ in range(n_iter):
        bounds = [-1e9] + [(c[k - 1] + c[k]) / 2 for k in range(1, n)] + [1e9]
        nc = []
        for k in range(n):
            a, b = bounds[k] / sigma, bounds[k + 1] / sigma
            mass = 0.5 * (1 + math.erf(b / s2)) - 0.5 * (1 + math.erf(a / s2))
            if mass < 1e-12:
                nc.append(c[k])
            else:
                pa = math.exp(-0.5 * a * a) / s2pi
                pb = math.exp(-0.5 * b * b) / s2pi
                nc.append((pa - pb) * sigma / mass)
        if max(abs(x - y) for x, y in zip(nc, c)) < 1e-9:
            break
        c = nc
    t = torch.tensor(c, dtype=torch.float32)
    _codebooks[key] = t
    return t


def stream_signs(layer_idx: int, hd: int) -> torch.Tensor:
    """Random +-1 signs of the stream rotation, cache.py:201-204 (CPU generator)."""
    g = torch.Generator(device="cpu").manual_seed(42 + layer_idx * 7919)
    return (torch.randint(0, 2, (hd,), generator=g) * 2 - 1).to(torch.float32)


# ---------------------------------------------------------------------------
# RoPE helpers (rope.py:8-47)
# ---------------------------------------------------------------------------
def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def rope_cos_sin(positions, inv_freq):
    """fp32 phases fl(theta_i * pos) duplicated over both halves (rope.py:13-18)."""
    freqs = positions.float()[:, None] * inv_freq.float()[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def undo_rope(keys, positions, inv_freq):
    cos, sin = rope_cos_sin(positions, inv_freq.to(keys.device))
    return keys * cos - rotate_half(keys) * sin


def get_rope_inv_freq(model):
    """model.model.rotary_emb.inv_freq (or the first layer's), else
    1/theta^(arange(0,hd,2)/hd) from the config (rope.py:32-47)."""
    backbone = getattr(model, "model", getattr(model, "transformer", None))
    layers = getattr(backbone, "layers", None) if backbone is not None else None
    for t in (backbone, layers[0] if layers is not None and len(layers) else None):
        if t is None:
            continue
        rot = getattr(t, "rotary_emb", None) or \
            getattr(getattr(t, "self_attn", None) or object(), "rotary_emb", None)
        if rot is not None and hasattr(rot, "inv_freq"):
            return rot.inv_freq.detach().float().cpu()
    cfg = model.config
    hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    theta = getattr(cfg, "rope_theta", 10000.0)
    rp = getattr(cfg, "rope_parameters", None)
    if isinstance(rp, dict) and "rope_theta" in rp:
        theta = rp["rope_theta"]
    return 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
