"""torch-tensor wrappers over the libshard_hip C ABI.

Every wrapper checks shapes/dtypes/devices on the host before calling into the
library (the kernels assume what is checked here), passes raw device pointers
and the current HIP stream, and raises ShardHipError on a non-zero status.
Tensors must live on a ROCm device; there is no CPU path.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import DecodeArgs, ShardHipError, ShardHipUnavailable  # noqa: F401


def _require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ShardHipUnavailable(
                "shard_amd kernels run on the GPU only (got a tensor on %s)" % t.device)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t):
    """The current stream of t's device: torch's raw stream query (the handle
    torch.cuda.current_stream(t.device).cuda_stream returns, without building
    a Stream object on every call)."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.get_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


ERR_WORKSPACE = -4  # SHARD_ERR_WORKSPACE of include/shard_hip.h


def _contig(t, dtype, name):
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    return t if t.is_contiguous() else t.contiguous()


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# prefill compression: keys
# ---------------------------------------------------------------------------
def pca_project(a: torch.Tensor, bt: torch.Tensor) -> torch.Tensor:
    """C = A @ Bt^T on MFMA; A (m, k) fp16, Bt (n, k) fp16 -> (m, n) fp32."""
    _require_gpu(a, bt)
    lib = _lib.load()
    a = _contig(a, torch.float16, "a")
    bt = _contig(bt, torch.float16, "bt")
    m, k = a.shape
    n, k2 = bt.shape
    if k != k2:
        raise ValueError("pca_project: inner dims differ")
    c = torch.empty(m, n, dtype=torch.float32, device=a.device)
    _lib.check("shard_pca_project", lib.shard_pca_project(
        _p(a), m, k, k, _p(bt), n, _p(c), n, _stream(a)))
    return c


def pca_project_f32(a: torch.Tensor, bt: torch.Tensor) -> torch.Tensor:
    """C = A @ Bt^T on fp32 MFMA; A (m, k) fp32, Bt (n, k) fp32 -> (m, n) fp32
    (the reference's fp32 projection, cache.py:389-392)."""
    _require_gpu(a, bt)
    lib = _lib.load()
    a = _contig(a, torch.float32, "a")
    bt = _contig(bt, torch.float32, "bt")
    m, k = a.shape
    n, k2 = bt.shape
    if k != k2:
        raise ValueError("pca_project_f32: inner dims differ")
    c = torch.empty(m, n, dtype=torch.float32, device=a.device)
    _lib.check("shard_pca_project_f32", lib.shard_pca_project_f32(
        _p(a), m, k, k, _p(bt), n, _p(c), n, _stream(a)))
    return c


def rope_phases(start: int, n: int, inv_freq: torch.Tensor) -> torch.Tensor:
    """(n, hd/2, 2) fp32 (cos, sin) of fl((start + t) * inv_freq[i])."""
    _require_gpu(inv_freq)
    lib = _lib.load()
    inv_freq = _contig(inv_freq, torch.float32, "inv_freq")
    hd2 = inv_freq.numel()
    out = torch.empty(n, hd2, 2, dtype=torch.float32, device=inv_freq.device)
    _lib.check("shard_rope_phases", lib.shard_rope_phases(start, n, hd2, _p(inv_freq), _p(out),
                                                          _stream(inv_freq)))
    return out


_ROPE_K_ORDER = {}


def rope_k_order(n_kv: int) -> torch.Tensor:
    """Basis column of each k position of shard_pca_project_rope's permuted k
    order (head_dim 128): k = 64 c + 16 s + 8 hh + e with chunk c = head c // 2,
    pair half c % 2, step s = 2 j + o, element e -> dim d0 + 4 o + e (e < 4)
    or 64 + d0 + 4 o + e - 4, d0 = 32 (c % 2) + 16 j + 8 hh."""
    order = _ROPE_K_ORDER.get(n_kv)
    if order is None:
        cols = []
        for c in range(2 * n_kv):
            g, ph = divmod(c, 2)
            for s in range(4):
                j, o = divmod(s, 2)
                for hh in range(2):
                    d0 = 32 * ph + 16 * j + 8 * hh
                    for e in range(8):
                        d = d0 + 4 * o + e if e < 4 else 64 + d0 + 4 * o + e - 4
                        cols.append(g * 128 + d)
        order = torch.tensor(cols, dtype=torch.long)
        _ROPE_K_ORDER[n_kv] = order
    return order


def rope_basis(bt: torch.Tensor) -> torch.Tensor:
    """The basis bt (n, G*128) fp16 with its columns in pca_project_rope's k order."""
    G = bt.shape[1] // 128
    return _contig(bt, torch.float16, "bt")[:, rope_k_order(G).to(bt.device)].contiguous()


def pca_project_rope(k: torch.Tensor, start: int, n_comp: int, phases: torch.Tensor,
                     btp: torch.Tensor, bias=None) -> torch.Tensor:
    """undo-RoPE of post-RoPE keys k (B, G, T, 128) fp16 at positions start +
    t, times the basis: (B*n_comp, n) fp32 = fp16(undo(k)) @ bt^T - bias, with
    btp = rope_basis(bt) for bt (n, G*128) fp16 and the undo in k_prepare's
    arithmetic (phases from rope_phases); one launch, no operand round trip."""
    _require_gpu(k, phases, btp)
    lib = _lib.load()
    k = _contig(k, torch.float16, "k")
    B, G, T, D = k.shape
    phases = _contig(phases, torch.float32, "phases")
    n = btp.shape[0]
    if btp.shape[1] != G * D or phases.shape[0] < n_comp:
        raise ValueError("pca_project_rope: basis or phase table does not match the keys")
    btp = _contig(btp, torch.float16, "btp")
    if bias is not None:
        bias = _contig(bias, torch.float32, "bias")
    c = torch.empty(B * n_comp, n, dtype=torch.float32, device=k.device)
    _lib.check("shard_pca_project_rope", lib.shard_pca_project_rope(
        _p(k), B, G, T, D, start, n_comp, _p(phases), _p(btp), n,
        _p(bias) if bias is not None else None, _p(c), n, _stream(k)))
    return c


def k_prepare(k: torch.Tensor, start: int, n_comp: int, inv_freq: torch.Tensor,
              mean: torch.Tensor, out_dtype=torch.float16) -> torch.Tensor:
    """undo-RoPE + mean subtraction of keys (B, G, T, D) fp16 -> (B*n_comp, G*D)
    rows in out_dtype: fp16 (the fp16 GEMM operand) or fp32 (no rounding)."""
    _require_gpu(k, inv_freq, mean)
    lib = _lib.load()
    k = _contig(k, torch.float16, "k")
    B, G, T, D = k.shape
    inv_freq = _contig(inv_freq.to(k.device), torch.float32, "inv_freq")
    mean = _contig(mean, torch.float32, "mean")
    out = torch.empty(B * n_comp, G * D, dtype=out_dtype, device=k.device)
    if out_dtype == torch.float16:
        fn, name = lib.shard_k_prepare, "shard_k_prepare"
    elif out_dtype == torch.float32:
        fn, name = lib.shard_k_prepare_f32, "shard_k_prepare_f32"
    else:
        raise TypeError(f"k_prepare: out_dtype must be float16 or float32, got {out_dtype}")
    _lib.check(name, fn(_p(k), B, G, T, D, start, n_comp, _p(inv_freq), _p(mean), _p(out), _stream(k)))
    return out


def int4_quant_pack(proj: torch.Tensor, bits: torch.Tensor, want_codes: bool = False):
    """Group quant -> dequant -> int4 -> packed (bit-exact chain).

    proj (n, keep) fp32; bits (keep,) int32.  Returns dict(packed, coeff_scale,
    lo, rng[, codes])."""
    _require_gpu(proj)
    lib = _lib.load()
    proj = _contig(proj, torch.float32, "proj")
    bits = torch.as_tensor(bits, dtype=torch.int32).to(proj.device).contiguous()
    n, keep = proj.shape
    if bits.numel() != keep:
        raise ValueError("int4_quant_pack: bits length != keep")
    dev = proj.device
    packed = torch.empty((n * keep + 1) // 2, dtype=torch.uint8, device=dev)
    cs = torch.empty(keep, dtype=torch.float32, device=dev)
    lo = torch.empty(keep, dtype=torch.float32, device=dev)
    rng = torch.empty(keep, dtype=torch.float32, device=dev)
    codes = torch.empty(n, keep, dtype=torch.uint8, device=dev) if want_codes else None
    ws = _workspace(lib.shard_int4_quant_pack_workspace(n, keep), dev)
    _lib.check("shard_int4_quant_pack", lib.shard_int4_quant_pack(
        _p(proj), n, keep, _p(bits), _p(packed), _p(cs), _p(lo), _p(rng), _p(codes),
        _p(ws), ws.numel(), _stream(proj)))
    out = {"packed": packed, "coeff_scale": cs, "lo": lo, "rng": rng}
    if want_codes:
        out["codes"] = codes
    return out


# ---------------------------------------------------------------------------
# prefill compression: values
# ---------------------------------------------------------------------------
def fwht(x: torch.Tensor) -> torch.Tensor:
    """Normalized Walsh-Hadamard transform over the last dim (fp32, bit-exact)."""
    _require_gpu(x)
    lib = _lib.load()
    x = _contig(x, torch.float32, "x")
    d = x.shape[-1]
    y = torch.empty_like(x)
    _lib.check("shard_fwht", lib.shard_fwht(_p(x), _p(y), x.numel() // d, d, _stream(x)))
    return y


def vq_prepare(v: torch.Tensor, group_size: int = 4):
    """hadamard(fp32(v)) -> per-(bh, channel) abs max -> normalized subvectors.

    v: (B, G, T, D) fp16 or a (bh, seq, D) view whose last two dims are
    contiguous.  Returns (x (bh*seq*D/gs, gs) fp32, ch fp32 (bh, D), ch fp16)."""
    _require_gpu(v)
    lib = _lib.load()
    if v.dtype != torch.float16:
        raise TypeError("vq_prepare: v must be fp16")
    D = v.shape[-1]
    seq = v.shape[-2]
    v3 = v.reshape(-1, seq, D) if v.dim() != 3 else v
    if v3.stride(-1) != 1 or v3.stride(-2) != D:
        v3 = v3.contiguous()
    bh = v3.shape[0]
    dev = v.device
    x = torch.empty(bh * seq * D // group_size, group_size, dtype=torch.float32, device=dev)
    ch32 = torch.empty(bh, D, dtype=torch.float32, device=dev)
    ch16 = torch.empty(bh, D, dtype=torch.float16, device=dev)
    ws = _workspace(lib.shard_vq_prepare_workspace(bh, D), dev)
    _lib.check("shard_vq_prepare", lib.shard_vq_prepare(
        _p(v3), bh, seq, D, v3.stride(0), _p(x), _p(ch32), _p(ch16), _p(ws), ws.numel(),
        _stream(v)))
    return x, ch32, ch16


def vq_assign(x: torch.Tensor, centroids: torch.Tensor) -> torch.Tensor:
    """argmin_k ||x - c_k||^2 (direct fp32 form, first index on ties) -> int32."""
    _require_gpu(x, centroids)
    lib = _lib.load()
    x = _contig(x, torch.float32, "x")
    c = _contig(centroids, torch.float32, "centroids")
    n, d = x.shape
    idx = torch.empty(n, dtype=torch.int32, device=x.device)
    _lib.check("shard_vq_assign", lib.shard_vq_assign(
        _p(x), n, d, _p(c), c.shape[0], _p(idx), _stream(x)))
    return idx


VQ_TABLE_BINS = 16  # cells per dim of the candidate table over [-1, 1]^4
# Rows from which k-means assigns through a candidate table rebuilt every
# iteration: measured on MI355X at 8.4M and 67M normalized rows, the table
# assigns in 10-11 ps per row against 32 for the all-centroid kernel, and a
# build (16^4 cells) takes about 0.1 ms.
VQ_TABLE_MIN_ROWS = 6_000_000


class VqTable:
    """Candidate table of one codebook (shard_vq_table_build): the box
    [lo, hi]^4 in nbins^4 cells, each listing the centroids that can be a
    row's nearest there.  Valid for the centroids it was built from."""

    def __init__(self, centroids: torch.Tensor, lo: float = -1.0, hi: float = 1.0,
                 nbins: int = VQ_TABLE_BINS):
        _require_gpu(centroids)
        lib = _lib.load()
        c = _contig(centroids, torch.float32, "centroids")
        if c.dim() != 2 or c.shape[1] != 4:
            raise ValueError("VqTable: centroids must be (k, 4)")
        self.k, self.lo, self.hi, self.nbins = c.shape[0], float(lo), float(hi), int(nbins)
        nbytes = lib.shard_vq_table_bytes(self.k, self.nbins)
        if nbytes == 0:
            raise ValueError(f"VqTable: unsupported k={self.k} or nbins={self.nbins}")
        self.table = torch.empty(nbytes, dtype=torch.uint8, device=c.device)
        self.centroids = c
        _lib.check("shard_vq_table_build", lib.shard_vq_table_build(
            _p(c), self.k, self.lo, self.hi, self.nbins, _p(self.table), nbytes, _stream(c)))

    @staticmethod
    def supported(centroids: torch.Tensor) -> bool:
        k = centroids.shape[0]
        return centroids.dim() == 2 and centroids.shape[1] == 4 and k % 32 == 0 and 0 < k <= 256


def vq_undecided_rows(ws: torch.Tensor, n: int) -> int:
    """Rows that the last table assignment of n rows into workspace ws left to
    the all-centroid scan: the per-wave counts at the workspace's start (one
    per wave of a launch of min(ceil(ceil(n / 64) / 4), 4096) workgroups of 4
    waves)."""
    groups = (n + 63) // 64
    nwaves = 4 * min((groups + 3) // 4, 4096)
    return int(ws[:4 * nwaves].view(torch.int32).sum().item())


def vq_assign_table(x: torch.Tensor, table: "VqTable", ws=None) -> torch.Tensor:
    """vq_assign(x, table.centroids) through the table (same result)."""
    _require_gpu(x)
    lib = _lib.load()
    x = _contig(x, torch.float32, "x")
    n = x.shape[0]
    if x.dim() != 2 or x.shape[1] != 4:
        raise ValueError("vq_assign_table: x must be (n, 4)")
    idx = torch.empty(n, dtype=torch.int32, device=x.device)
    need = lib.shard_vq_assign_table_workspace(n)
    if ws is None or ws.numel() < need:
        ws = _workspace(need, x.device)
    _lib.check("shard_vq_assign_table", lib.shard_vq_assign_table(
        _p(x), n, _p(table.centroids), table.k, _p(table.table), table.table.numel(), table.nbins,
        table.lo, table.hi, _p(idx), _p(ws), ws.numel(), _stream(x)))
    return idx


def _vq_rows(v: torch.Tensor):
    """(bh, seq, D) view of V whose last two dims are contiguous."""
    if v.dtype != torch.float16:
        raise TypeError("V must be fp16")
    D, seq = v.shape[-1], v.shape[-2]
    v3 = v.reshape(-1, seq, D) if v.dim() != 3 else v
    if v3.stride(-1) != 1 or v3.stride(-2) != D:
        v3 = v3.contiguous()
    return v3


def vq_scales(v: torch.Tensor):
    """shard_vq_prepare's channel scales alone: (ch fp32 (bh, D), ch fp16,
    their reciprocals fp32)."""
    _require_gpu(v)
    lib = _lib.load()
    v3 = _vq_rows(v)
    bh, seq, D = v3.shape
    dev = v.device
    ch32 = torch.empty(bh, D, dtype=torch.float32, device=dev)
    ch16 = torch.empty(bh, D, dtype=torch.float16, device=dev)
    rcp = torch.empty(bh, D, dtype=torch.float32, device=dev)
    ws = _workspace(lib.shard_vq_prepare_workspace(bh, D), dev)
    _lib.check("shard_vq_scales", lib.shard_vq_scales(
        _p(v3), bh, seq, D, v3.stride(0), _p(ch32), _p(ch16), _p(rcp), _p(ws), ws.numel(),
        _stream(v)))
    return ch32, ch16, rcp


def vq_encode_table(v: torch.Tensor, ch32: torch.Tensor, rcp: torch.Tensor, table: "VqTable",
                    ws=None) -> torch.Tensor:
    """Indices of V's normalized subvectors (head_dim 128) through the table,
    formed from V in registers: vq_assign_table(vq_prepare(v)[0], table)."""
    _require_gpu(v, ch32, rcp)
    lib = _lib.load()
    v3 = _vq_rows(v)
    bh, seq, D = v3.shape
    n = bh * seq * (D // 4)
    idx = torch.empty(n, dtype=torch.int32, device=v.device)
    need = lib.shard_vq_encode_table_workspace(n)
    if ws is None or ws.numel() < need:
        ws = _workspace(need, v.device)
    ch32 = _contig(ch32, torch.float32, "ch")
    rcp = _contig(rcp, torch.float32, "rcp")
    _lib.check("shard_vq_encode_table", lib.shard_vq_encode_table(
        _p(v3), bh, seq, D, v3.stride(0), _p(ch32), _p(rcp), _p(table.centroids), table.k,
        _p(table.table), table.table.numel(), table.nbins, table.lo, table.hi, _p(idx), _p(ws),
        ws.numel(), _stream(v)))
    return idx


def kmeans_update(x: torch.Tensor, idx: torch.Tensor, centroids: torch.Tensor, ws=None):
    """One deterministic k-means update; returns (new_centroids, max_delta (1,) fp32)."""
    _require_gpu(x, idx, centroids)
    lib = _lib.load()
    x = _contig(x, torch.float32, "x")
    idx = _contig(idx, torch.int32, "idx")
    c = _contig(centroids, torch.float32, "centroids")
    n, d = x.shape
    k = c.shape[0]
    newc = torch.empty_like(c)
    maxd = torch.empty(1, dtype=torch.float32, device=x.device)
    need = lib.shard_kmeans_update_workspace_d(n, k, d)
    if ws is None or ws.numel() < need:
        ws = _workspace(need, x.device)
    _lib.check("shard_kmeans_update", lib.shard_kmeans_update(
        _p(x), n, d, _p(idx), _p(c), k, _p(newc), _p(maxd), _p(ws), ws.numel(), _stream(x)))
    return newc, maxd


_init_rows = {}


# torch's CPU randperm below this size: a forward Fisher-Yates shuffle of
# 0..n-1 where step i swaps entry i with entry i + (random() % (n - i)),
# random() being the generator's next 32-bit MT19937 output
_RANDPERM_SHUFFLE_MAX = (2**32 - 1) // 20


def _randperm_head(n: int, k: int, seed: int) -> torch.Tensor:
    """The first k entries of torch.randperm(n) from a CPU generator seeded
    with `seed`, without building the n-entry permutation.  The shuffle fixes
    entry i at step i, so k steps decide the first k entries; they are replayed
    on a sparse map of the swapped entries.  The generator is MT19937 seeded
    like the standard init_genrand(seed), whose 32-bit outputs numpy's legacy
    RandomState reproduces.  Sizes or seeds outside that form fall back to
    torch.randperm."""
    if not (0 < n < _RANDPERM_SHUFFLE_MAX and 0 <= seed < 2**32):
        g = torch.Generator(device="cpu").manual_seed(seed)
        return torch.randperm(n, generator=g)[:k].clone()
    steps = min(k, n - 1)
    raw = np.random.RandomState(seed).randint(0, 2**32, size=max(steps, 0), dtype=np.uint64)
    moved = {}
    out = []
    for i in range(min(k, n)):
        if i < n - 1:
            z = i + int(raw[i]) % (n - i)
            a, b = moved.get(i, i), moved.get(z, z)
            moved[i], moved[z] = b, a
        out.append(moved.get(i, i))
    return torch.tensor(out, dtype=torch.int64)


def _kmeans_init_rows(n: int, k: int, seed: int) -> torch.Tensor:
    """First k entries of randperm(n) from a CPU generator seeded with `seed`
    (cache.py:21-26), kept per (n, k, seed): every layer of a cache draws with
    the same seed, so the rows repeat for equal n."""
    key = (int(n), int(k), int(seed))
    rows = _init_rows.get(key)
    if rows is None:
        rows = _randperm_head(int(n), int(k), int(seed))
        if len(_init_rows) > 64:
            _init_rows.clear()
        _init_rows[key] = rows
    return rows


def kmeans(data: torch.Tensor, k: int, n_iter: int = 30, seed: int = 42):
    """k-means of cache.py:21-39 on the GPU: CPU-generator randperm init, then
    assign (shard_vq_assign, or through a candidate table for large d = 4
    sets: the same indices) + deterministic update per iteration; stops like the
    reference (max |delta| < 1e-4 once it >= 5) and returns the last assignment
    (made against the pre-update centroids) with the final centroids."""
    n, d = data.shape
    perm = _kmeans_init_rows(n, k, seed).to(data.device)
    centroids = data[perm].clone()
    lib = _lib.load()
    ws = _workspace(lib.shard_kmeans_update_workspace_d(n, centroids.shape[0], d), data.device)
    # the rows are shard_vq_prepare's normalized subvectors (in [-1, 1]); at
    # this size a candidate table per iteration pays for its build
    tab_ws = None
    if n >= VQ_TABLE_MIN_ROWS and VqTable.supported(centroids):
        tab_ws = _workspace(lib.shard_vq_assign_table_workspace(n), data.device)
    idx = None
    deltas = []
    for it in range(n_iter):
        if tab_ws is not None:
            idx = vq_assign_table(data, VqTable(centroids), tab_ws)
        else:
            idx = vq_assign(data, centroids)
        new, maxd = kmeans_update(data, idx, centroids, ws)
        deltas.append(maxd)
        # one host sync per iteration, as the reference's .item() (cache.py:36)
        if it >= 5 and maxd.item() < 1e-4:
            centroids = new
            break
        centroids = new
    return centroids, idx


# ---------------------------------------------------------------------------
# decode stream
# ---------------------------------------------------------------------------
def stream_quant(x: torch.Tensor, signs: torch.Tensor, codebook: torch.Tensor,
                 with_deq: bool = False, qjl: bool = False):
    """Per-token Lloyd-Max quantizer; x (..., D) fp16 -> (idx u8 (..., D), norm fp16 (...)
    [, qsign u8 (..., D), qscale fp16 (...) with qjl] [, deq fp16 (..., D) = the token
    as the reference dequantizes it])."""
    _require_gpu(x, signs, codebook)
    x = _contig(x, torch.float16, "x")
    idx = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    norm = torch.empty(x.shape[:-1], dtype=torch.float16, device=x.device)
    qs = torch.empty(x.shape, dtype=torch.uint8, device=x.device) if qjl else None
    qsc = torch.empty(x.shape[:-1], dtype=torch.float16, device=x.device) if qjl else None
    deq = torch.empty(x.shape, dtype=torch.float16, device=x.device) if with_deq else None
    stream_quant_into(x, signs, codebook, idx, norm, deq, qs, qsc)
    out = (idx, norm) + ((qs, qsc) if qjl else ())
    return out + (deq,) if with_deq else out


def stream_quant_into(x, signs, codebook, idx_out, norm_out, deq_out=None, qsign_out=None,
                      qscale_out=None):
    lib = _lib.load()
    D = x.shape[-1]
    rows = x.numel() // D
    _lib.check("shard_stream_quant", lib.shard_stream_quant_qjl(
        _p(x), rows, D, _p(signs), _p(codebook), codebook.numel(), _p(idx_out), _p(norm_out),
        _p(qsign_out), _p(qscale_out), _p(deq_out), _stream(x)))


def stream_quant_kv_at(k, v, signs, codebook, k_idx, k_norm, k_deq, v_idx, v_norm, v_deq,
                       k_qsign=None, k_qscale=None, v_qsign=None, v_qscale=None):
    """One decode token's K and V (contiguous fp16 (..., D), same shape) quantized
    by one launch into outputs given as device addresses (ints): the rows of the
    cache's stream buffers (cache.py:207-215)."""
    lib = _lib.load()
    D = k.shape[-1]
    _lib.check("shard_stream_quant_kv", lib.shard_stream_quant_kv(
        k.data_ptr(), v.data_ptr(), k.numel() // D, D, signs.data_ptr(), codebook.data_ptr(),
        codebook.numel(), k_idx, k_norm, k_deq, v_idx, v_norm, v_deq, k_qsign, k_qscale,
        v_qsign, v_qscale, _stream(k)))


def rope_stream_append_at(q, k, v, cos, sin, signs, codebook, q_out, k_idx, k_norm, k_deq,
                          v_idx, v_norm, v_deq, k_qsign=None, k_qscale=None, v_qsign=None,
                          v_qscale=None, row_dev=None, row_cap=0):
    """RoPE of q and k (transformers' fp16 arithmetic) and the rotated k and v
    appended to the stream in one launch.  q (B, H, D), k and v (B, G, D):
    contiguous fp16; cos and sin (B, D) or (1, D) (shared by the batch),
    contiguous fp16; q_out (B, H, D) fp16; the stream outputs are device
    addresses (ints) of this token's rows, or, with row_dev (a one-element
    int32 tensor on q's device), of the buffers' first rows: the token then
    goes to row row_dev[0] (written only when it is below row_cap), read at
    run time, so a captured graph appends every step's token."""
    lib = _lib.load()
    B, H, D = q.shape
    G = k.shape[1]
    if cos.shape != sin.shape or cos.shape[-1] != D or cos.shape[0] not in (1, B):
        raise ValueError(f"cos/sin {tuple(cos.shape)} do not fit q {tuple(q.shape)}")
    cs_stride = 0 if cos.shape[0] == 1 else D
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(), cs_stride,
            B, H, G, D,
            q_out.data_ptr(), signs.data_ptr(), codebook.data_ptr(), codebook.numel(),
            k_idx, k_norm, k_deq, v_idx, v_norm, v_deq, k_qsign, k_qscale, v_qsign, v_qscale)
    if row_dev is None:
        _lib.check("shard_rope_stream_append", lib.shard_rope_stream_append(*args, _stream(q)))
        return
    if row_dev.dtype != torch.int32 or row_dev.device != q.device or row_dev.numel() < 1:
        raise TypeError("row_dev must be an int32 tensor on q's device")
    _lib.check("shard_rope_stream_append_dev", lib.shard_rope_stream_append_dev(
        *args, row_dev.data_ptr(), int(row_cap), _stream(q)))


def stream_dequant(idx: torch.Tensor, norm: torch.Tensor, signs: torch.Tensor,
                   codebook: torch.Tensor, qsign: torch.Tensor = None,
                   qscale: torch.Tensor = None) -> torch.Tensor:
    """fp16(fp16(H(cb[idx] (+ (2 qsign - 1) qscale)) * signs) * norm) for (..., D) codes."""
    _require_gpu(idx, norm, signs, codebook)
    lib = _lib.load()
    idx = _contig(idx, torch.uint8, "idx")
    norm = _contig(norm, torch.float16, "norm")
    if qsign is not None:
        qsign = _contig(qsign, torch.uint8, "qsign")
        qscale = _contig(qscale, torch.float16, "qscale")
    D = idx.shape[-1]
    y = torch.empty(idx.shape, dtype=torch.float16, device=idx.device)
    _lib.check("shard_stream_dequant", lib.shard_stream_dequant_qjl(
        _p(idx), _p(norm), _p(qsign), _p(qscale), idx.numel() // D, D, _p(signs),
        _p(codebook), _p(y), _stream(idx)))
    return y


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------
class DecodeCall:
    """The ctypes argument block of one layer's decode call and the tensors it
    points to.  A layer keeps one and refreshes the per-step fields
    (``refresh``), so a decode step sets a dozen fields instead of rebuilding
    the block."""

    def __init__(self, args: DecodeArgs, static: list):
        self.args = args
        self.static = static     # the layer format's tensors
        self.step = []           # this step's q, out, mask, ... (set by refresh)
        self.out = None

    @property
    def keep(self):
        return self.static + self.step

    def workspace_bytes(self) -> int:
        """The library's workspace size for the block as it stands: asked on
        every call, since it depends on every count the split choice reads
        (context, extra tokens, batch, requested splits)."""
        return int(_lib.load().shard_decode_attn_workspace(ctypes.byref(self.args)))


def decode_supported(head_dim: int, n_q_heads: int, n_kv_heads: int, rank_pad: int) -> bool:
    """The shapes shard_decode_attn takes (its shard_decode_supported): head_dim
    128 with up to 64 query heads per kv head, or head_dim 64 with an even
    number of kv heads (run in pairs as 128-dim heads) and up to 32 query heads
    per kv head; rank a multiple of 32 up to 256.  Other layers run the
    reference's unfused path (fp16 K/V rebuilt by shard_kv_reconstruct,
    attention.py:411)."""
    if head_dim not in (64, 128) or n_kv_heads <= 0 or n_q_heads <= 0 or n_q_heads % n_kv_heads:
        return False
    g = n_q_heads // n_kv_heads
    if head_dim == 64:
        if n_kv_heads % 2:
            return False
        g *= 2  # query heads per pair
    return g <= 64 and 0 < rank_pad <= 256 and rank_pad % 32 == 0


# The decode kernels fold the mean and the offsets of their nibble decoding
# into one constant k-step: C = 16 mean - 16512 sum_{even r} A'(r) - 1152
# sum_{odd r} A'(r) per key dim, A' = fp16(basis * coeff_scale), held as 16
# bf16 parts (shard_decode_prepare): any finite magnitude the fp32
# accumulators hold.  A layer whose C is not finite or beyond this bound
# (non-finite basis or scales) takes the unfused path.
DECODE_CONSTANT_LIMIT = 1e30


def decode_constant_max(basis: torch.Tensor, coeff_scale: torch.Tensor, mean: torch.Tensor) -> float:
    """max |C| over the key dims of a layer (float64, as shard_decode_prepare
    accumulates it): basis (G*D, rank) fp16, coeff_scale (rank) fp16, mean (G*D)."""
    a = (basis.float() * coeff_scale.float()[None, :]).half().double()
    w = torch.where(torch.arange(a.shape[1], device=a.device) % 2 == 0, 16512.0, 1152.0).double()
    c = 16.0 * mean.double() - a @ w
    return float(c.abs().max())


def decode_prepare(fmt) -> torch.Tensor:
    """Per-layer constant operands of the decode kernel (uint8 buffer on the device)."""
    lib = _lib.load()
    basis, cs, mean = fmt["k_basis_pad"], fmt["k_coeff_scale_pad"], fmt["k_mean_f16"]
    _require_gpu(basis, cs, mean)
    G, rank = fmt["n_kv"], fmt["rank_pad"]
    inv = fmt["inv_freq_dev"]
    images = G // 2 if fmt["head_dim"] == 64 else G  # head_dim 64: one image per pair of kv heads
    buf = torch.empty(lib.shard_decode_prepare_bytes(images, rank), dtype=torch.uint8,
                      device=basis.device)
    _lib.check("shard_decode_prepare", lib.shard_decode_prepare(
        _p(basis), _p(cs), _p(mean), _p(inv), G, fmt["head_dim"], rank, _p(buf), buf.numel(),
        _stream(basis)))
    return buf


def additive_mask(mask: torch.Tensor) -> torch.Tensor:
    """An attention mask as the fp32 additive form the decode kernel reads:
    a boolean mask (True = attend, what transformers builds for its sdpa
    attention) becomes 0 / the fp32 minimum, as transformers' own float masks
    hold them; a float mask is taken as added to the scores."""
    if mask.dtype == torch.bool:
        return torch.zeros(mask.shape, dtype=torch.float32, device=mask.device).masked_fill_(
            ~mask, torch.finfo(torch.float32).min)
    return mask if mask.dtype == torch.float32 else mask.float()


def make_decode_args(q, fmt, pos_q, inv_freq, mask=None, n_splits=0, out=None,
                     stream_n=0, decode_kv=None, stream_n_dev=None) -> DecodeCall:
    """Build shard_decode_args for one layer.

    q (B, H, D) fp16 (post-RoPE); ``fmt`` is the layer's device format dict
    (see cache.CompressedLayerFormat); decode_kv = (dec_k, dec_v) fp16
    (B, G, S, D) or None.  ``pos_q`` is an int, or an int64 tensor on q's
    device whose last element the kernel reads (no host read-back).  With
    ``stream_n_dev`` (a one-element int32 tensor on q's device) the call
    attends over its value's worth of stream rows, at most stream_n."""
    _require_gpu(q)
    B, H, D = q.shape
    # the fused kernel's codebook: 4-value subvectors, 256 rows (padded);
    # other shapes only reach kv_reconstruct, which takes the codebook as is
    cb = fmt.get("v_centroids_pad")
    if cb is None:
        cb = fmt["v_centroids_f16"]
    keep = []
    a = DecodeArgs()
    a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim = B, H, fmt["n_kv"], D
    a.rank, a.n_comp = fmt["rank_pad"], fmt["n_compress"]
    a.compress_start = fmt["compress_start"]
    for name, t in (("inv_freq", fmt["inv_freq_dev"]), ("k_coeffs", fmt["k_coeffs_pad"]),
                    ("k_coeff_scale", fmt["k_coeff_scale_pad"]), ("k_basis", fmt["k_basis_pad"]),
                    ("k_mean", fmt["k_mean_f16"]), ("prep", fmt.get("decode_prep")),
                    ("v_idx", fmt["v_indices"]),
                    ("v_codebook", cb), ("v_ch", fmt["v_ch_f16"]),
                    ("sink_k", fmt["sink_k"]), ("sink_v", fmt["sink_v"]),
                    ("win_k", fmt["win_k"]), ("win_v", fmt["win_v"])):
        if t is None:  # no decode operands: a layer shape only kv_reconstruct takes
            setattr(a, name, None)
            continue
        setattr(a, name, t.data_ptr())
        keep.append(t)
    a.n_sink = fmt["sink_k"].shape[2]
    a.n_win = fmt["win_k"].shape[2]
    a.v_codebook_n, a.v_group = cb.shape
    call = DecodeCall(a, keep)
    return call.refresh(q, fmt, pos_q, inv_freq, mask, n_splits, out, stream_n, decode_kv,
                        stream_n_dev)


def _decode_refresh(self, q, fmt, pos_q, inv_freq=None, mask=None, n_splits=0, out=None,
                    stream_n=0, decode_kv=None, stream_n_dev=None):
    """Point this call at one step's q, position, stream, decode tokens and mask
    (the fields that change between decode steps; the layer's format pointers
    stay).  Returns self; self.out is the (B, H, D) fp16 output tensor."""
    _require_gpu(q)
    if q.dtype != torch.float16 or not q.is_contiguous():
        raise TypeError("q must be contiguous fp16 (B, H, D)")
    a = self.args
    B, H, D = q.shape
    if (B, H, D) != (a.batch, a.n_q_heads, a.head_dim):
        raise ValueError(f"q shape {(B, H, D)} does not match the call's {(a.batch, a.n_q_heads, a.head_dim)}")
    step = [q]
    a.q = q.data_ptr()
    if isinstance(pos_q, torch.Tensor):
        if pos_q.dtype != torch.int64 or pos_q.device != q.device or pos_q.numel() < 1:
            raise TypeError("a device pos_q must be a non-empty int64 tensor on q's device")
        pos_t = pos_q.reshape(-1)[-1:]
        a.pos_q, a.pos_q_dev = 0, pos_t.data_ptr()
        step.append(pos_t)
    else:
        a.pos_q, a.pos_q_dev = int(pos_q), None
    inv = fmt["inv_freq_dev"] if inv_freq is None else inv_freq
    a.inv_freq = inv.data_ptr()
    step.append(inv)
    if decode_kv is not None:
        dk, dv = decode_kv
        a.dec_k, a.dec_v = dk.data_ptr(), dv.data_ptr()
        a.n_dec, a.dec_stride = dk.shape[2], dk.shape[2]
        step += [dk, dv]
    else:
        a.dec_k = a.dec_v = None
        a.n_dec = a.dec_stride = 0
    if stream_n > 0:
        a.s_k, a.s_v = fmt["k_deq_buf"].data_ptr(), fmt["v_deq_buf"].data_ptr()
        step += [fmt["k_deq_buf"], fmt["v_deq_buf"]]
    else:
        a.s_k = a.s_v = None
    a.n_stream = stream_n
    if stream_n_dev is not None:
        if (stream_n_dev.dtype != torch.int32 or stream_n_dev.device != q.device
                or stream_n_dev.numel() < 1):
            raise TypeError("stream_n_dev must be an int32 tensor on q's device")
        a.n_stream_dev = stream_n_dev.data_ptr()
        step.append(stream_n_dev)
    else:
        a.n_stream_dev = None
    if mask is not None:
        m = additive_mask(mask).reshape(B, -1)
        n_total = (a.n_sink + a.n_comp + a.n_win + a.n_dec + a.n_stream)
        if m.shape[1] < n_total:
            raise ValueError(f"attention mask covers {m.shape[1]} keys, the cache holds {n_total}")
        if m.stride(-1) != 1:
            m = m.contiguous()
        a.mask, a.mask_stride = m.data_ptr(), m.stride(0)
        step.append(m)
    else:
        a.mask, a.mask_stride = None, 0
    if out is None:
        out = torch.empty(B, H, D, dtype=torch.float16, device=q.device)
    a.out = out.data_ptr()
    step.append(out)
    a.n_splits = int(n_splits)
    self.out = out
    self.step = step
    return self


DecodeCall.refresh = _decode_refresh


def decode_workspace(call: DecodeCall) -> torch.Tensor:
    """A decode workspace for ``call`` (zero-filled; reusable by later calls,
    one call at a time per buffer)."""
    need = call.workspace_bytes()
    return torch.zeros(max(need, 16), dtype=torch.uint8, device=call.out.device)


def decode_attn(call: DecodeCall, ws: torch.Tensor = None, allocate: bool = True) -> torch.Tensor:
    """Run the decode call; returns its (B, H, D) fp16 output.  A workspace ws
    that is missing or too small (the library checks before it launches
    anything) is replaced by a fresh one of the size the call needs, or, with
    allocate=False, raises ShardHipError with code SHARD_ERR_WORKSPACE."""
    lib = _lib.load()
    stream = _stream(call.out)
    if ws is not None:
        rc = lib.shard_decode_attn(ctypes.byref(call.args), ws.data_ptr(), ws.numel(), stream)
        if rc != ERR_WORKSPACE or not allocate:
            _lib.check("shard_decode_attn", rc)
            return call.out
    elif not allocate:
        raise _lib.ShardHipError("shard_decode_attn", ERR_WORKSPACE, "no workspace given")
    ws = decode_workspace(call)
    _lib.check("shard_decode_attn", lib.shard_decode_attn(
        ctypes.byref(call.args), ws.data_ptr(), ws.numel(), stream))
    return call.out


# SHARD_DECODE_NOALLOC_SCRATCH_BYTES of include/shard_hip.h
DECODE_NOALLOC_SCRATCH_BYTES = 8 << 20


def decode_attn_noalloc(call: DecodeCall) -> torch.Tensor:
    """The decode call through shard_decode_attn_noalloc: no workspace, no
    allocation (the library's per-GPU scratch holds the partial rows; calls
    that overlap on one GPU race on it).  Raises ShardHipError when the call's
    workspace would exceed DECODE_NOALLOC_SCRATCH_BYTES."""
    lib = _lib.load()
    _lib.check("shard_decode_attn_noalloc", lib.shard_decode_attn_noalloc(
        ctypes.byref(call.args), _stream(call.out)))
    return call.out


def bench_fp16_decode(q, k, v, n_splits=0, out=None, ws=None, seq=None):
    """The benchmark's same-GPU baseline: fp16 split-K GQA decode attention over
    uncompressed K/V (shard_bench_fp16_decode).  q (B, H, 128) with H = 4 G,
    k / v (B, G, T, 128) fp16 contiguous; n_splits 0 = two workgroups per CU.
    seq < T attends the first seq rows of each head (a preallocated cache)."""
    _require_gpu(q)
    lib = _lib.load()
    B, H, D = q.shape
    G, rows = k.shape[1], k.shape[2]
    T = rows if seq is None else int(seq)
    if D != 128 or H != 4 * G or tuple(k.shape) != (B, G, rows, D) or k.shape != v.shape:
        raise ValueError("bench_fp16_decode: q (B, 4G, 128), k/v (B, G, T, 128)")
    if not 0 < T <= rows:
        raise ValueError("bench_fp16_decode: seq must be in 1..T")
    for t in (q, k, v):
        if t.dtype != torch.float16 or not t.is_contiguous():
            raise ValueError("bench_fp16_decode takes contiguous fp16 tensors")
    if n_splits <= 0:
        cus = torch.cuda.get_device_properties(q.device).multi_processor_count
        n_splits = max(1, min((T + 31) // 32, 2 * cus // max(1, G * B)))
    if out is None:
        out = torch.empty(B, H, D, dtype=torch.float16, device=q.device)
    need = lib.shard_bench_fp16_decode_workspace(B, G, n_splits)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.check("shard_bench_fp16_decode", lib.shard_bench_fp16_decode_ld(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), B, G, T, rows, n_splits, out.data_ptr(),
        ws.data_ptr(), ws.numel(), _stream(q)))
    return out


def decode_workspace_bytes(call: DecodeCall) -> int:
    return call.workspace_bytes()


def kv_reconstruct(fmt, batch: int):
    """Full fp16 K (RoPE re-applied) and V of the compressed segment: (B, G, n, D)."""
    lib = _lib.load()
    dev = fmt["k_coeffs"].device
    B, G, n, D = batch, fmt["n_kv"], fmt["n_compress"], fmt["head_dim"]
    q_dummy = torch.empty(B, G * 4, D, dtype=torch.float16, device=dev)
    call = make_decode_args(q_dummy, fmt, 0, None)
    cb = fmt["v_centroids_f16"]  # its own shape: any group and codebook size the Cache takes
    call.args.v_codebook = cb.data_ptr()
    call.args.v_codebook_n, call.args.v_group = cb.shape
    call.args.k_coeffs = fmt["k_coeffs"].data_ptr()
    call.args.k_coeff_scale = fmt["k_coeff_scale"].data_ptr()
    call.args.k_basis = fmt["k_basis_f16"].data_ptr()
    call.args.rank = fmt["rank"]
    k_out = torch.empty(B, G, n, D, dtype=torch.float16, device=dev)
    v_out = torch.empty(B, G, n, D, dtype=torch.float16, device=dev)
    _lib.check("shard_kv_reconstruct", lib.shard_kv_reconstruct(
        ctypes.byref(call.args), _p(k_out), _p(v_out), _stream(k_out)))
    return k_out, v_out
