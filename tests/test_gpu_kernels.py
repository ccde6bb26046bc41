"""GPU parity of the integer/byte kernels against the CPU oracle (bit-exact),
and of the MFMA projection GEMM against an fp64 product of the same fp16 inputs."""
import numpy as np
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu


def _ops():
    from shard_amd import ops
    return ops


@pytest.mark.parametrize("want_codes", [True, False])
@pytest.mark.parametrize("n,alloc", [
    (5000, [4] * 64 + [2] * 64 + [8] * 64),
    (777, [6] * 64 + [0] * 64 + [2] * 32),
    (33, [8] * 10 + [4] * 6),
    (7, [3] * 20 + [0] * 5 + [5] * 10),  # odd element count: a padded last nibble
    (1, [2] * 32),
    (300, [4] * 30 + [2] * 12),          # even keep, not a multiple of 8: byte stores
    (2049, [1] * 8 + [7] * 56 + [4] * 64),  # constant, near-constant and one-sided columns
])
def test_int4_quant_pack_bitexact(cuda, n, alloc, want_codes):
    """Even keep takes two passes (column min/max, then codes and packing, the
    coefficient scale from each column's extreme elements); odd keep the
    three-pass chain.  Both bit-exact against the oracle's chain."""
    ops = _ops()
    keep = len(alloc)
    rng = np.random.default_rng(n)
    proj = (rng.standard_normal((n, keep)) * np.exp(-np.arange(keep) / 60.0)).astype(np.float32)
    if n > 2:
        proj[rng.integers(0, n, 3), rng.integers(0, keep, 3)] = 0.0
    if n == 2049:
        proj[:, 0] = 0.75                                            # constant: rng clamps to 1e-6
        proj[:, 1] = -3.0 + rng.random(n).astype(np.float32) * 4e-7   # range below 1e-6
        proj[:, 2] = np.abs(proj[:, 2]) + 5.0                        # all positive, lo far from 0
        proj[:, 3] = -np.abs(proj[:, 3]) - 5.0                       # all negative
    want = ref.k_code_chain(proj, alloc)
    got = ops.int4_quant_pack(torch.from_numpy(proj).to(cuda),
                              torch.tensor(alloc, dtype=torch.int32), want_codes=want_codes)
    assert np.array_equal(got["packed"].cpu().numpy(), want["packed"])
    assert np.array_equal(got["coeff_scale"].cpu().numpy(), want["coeff_scale"])
    if want_codes:
        assert np.array_equal(got["codes"].cpu().numpy(), want["codes"])
    nz = np.array(alloc) > 0
    assert np.array_equal(got["lo"].cpu().numpy()[nz], want["lo"][nz])
    assert np.array_equal(got["rng"].cpu().numpy()[nz], want["rng"][nz])


def test_int4_quant_pack_reference_golden(cuda, golden):
    """The HIP chain against the reference's own outputs (int4_chain.npz):
    group-quantizer ranges, coefficient scales and packed nibbles bit for bit,
    on .5-boundary columns of every width."""
    ops = _ops()
    g = golden("int4_chain.npz")
    alloc = [int(b) for b in g["alloc"]]
    got = ops.int4_quant_pack(torch.from_numpy(g["proj"]).to(cuda),
                              torch.tensor(alloc, dtype=torch.int32), want_codes=True)
    assert np.array_equal(got["packed"].cpu().numpy(), g["packed"])
    assert np.array_equal(got["coeff_scale"].cpu().numpy(), g["coeff_scale"])
    nz = np.array(alloc) > 0
    assert np.array_equal(got["lo"].cpu().numpy()[nz], g["lo"][nz])
    assert np.array_equal(got["rng"].cpu().numpy()[nz], g["rng"][nz])


@pytest.mark.parametrize("rows", [1, 16, 4099])
def test_stream_quant_bitexact(cuda, rows):
    ops = _ops()
    g = torch.Generator().manual_seed(rows)
    x = (torch.randn(rows, 128, generator=g) * torch.rand(rows, 1, generator=g) * 6).half()
    if rows > 3:
        x[1] = 0          # norm clamp path
        x[2, :5] = 60000  # large values
    cb = ref.lloyd_max_codebook(128, 8)
    signs = ref.stream_signs(11, 128)
    want_idx, want_n = ref.quantize_stream_token(x.numpy(), signs, cb)
    idx, nrm, deq = ops.stream_quant(x.to(cuda), torch.from_numpy(signs).to(cuda),
                                     torch.from_numpy(cb).to(cuda), with_deq=True)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(nrm.cpu().numpy().view(np.uint16), want_n.view(np.uint16))
    y = ops.stream_dequant(idx, nrm, torch.from_numpy(signs).to(cuda), torch.from_numpy(cb).to(cuda))
    want_y = ref.dequantize_stream_token(want_idx, want_n, signs, cb)
    got_y = y.cpu().numpy()
    fin = np.isfinite(want_n.astype(np.float32))
    gb, wb = got_y.view(np.uint16)[fin], want_y.view(np.uint16)[fin]
    bad = np.argwhere(gb != wb)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}: " \
        f"{gb[tuple(bad[:5].T)].tolist()} vs {wb[tuple(bad[:5].T)].tolist()}"
    # a norm that overflows fp16 (row 2) gives non-finite values on both sides
    assert np.array_equal(np.isfinite(got_y[~fin]), np.isfinite(want_y[~fin]))
    # the dequantized copy written at quantization time is the same
    got_d = deq.cpu().numpy()
    assert np.array_equal(got_d.view(np.uint16)[fin], want_y.view(np.uint16)[fin])


def _bits_eq(got, want):
    gb, wb = np.asarray(got).view(np.uint16), np.asarray(want).view(np.uint16)
    bad = np.argwhere(gb != wb)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:5].tolist()}"


@pytest.mark.parametrize("bits,qjl,hd", [
    (8, True, 128), (4, False, 128), (4, True, 128), (3, True, 128), (2, True, 128),
    (1, True, 128), (2, True, 64), (8, True, 256), (5, False, 256),
])
def test_stream_quant_widths_qjl_bitexact(cuda, bits, qjl, hd):
    """Lloyd-Max codes of 1..8 bits and the QJL residual (streaming.py:59-79):
    codes, norms, residual signs and fp16 scales, and both dequantizations."""
    ops = _ops()
    rows = 1031
    g = torch.Generator().manual_seed(bits * 1000 + hd)
    x = (torch.randn(rows, hd, generator=g) * torch.rand(rows, 1, generator=g) * 6).half()
    x[1] = 0
    cb = ref.lloyd_max_codebook(hd, bits)
    signs = ref.stream_signs(bits, hd)
    want = ref.quantize_stream_token(x.numpy(), signs, cb, qjl=qjl)
    sd, cd = torch.from_numpy(signs).to(cuda), torch.from_numpy(cb).to(cuda)
    got = ops.stream_quant(x.to(cuda), sd, cd, with_deq=True, qjl=qjl)
    got = [t.cpu().numpy() for t in got]
    assert np.array_equal(got[0], want[0])
    _bits_eq(got[1], want[1])
    if qjl:
        assert np.array_equal(got[2], want[2])
        _bits_eq(got[3], want[3])
    want_y = ref.dequantize_stream_token(want[0], want[1], signs, cb,
                                         *(want[2:4] if qjl else (None, None)))
    _bits_eq(got[-1], want_y)
    y = ops.stream_dequant(*(torch.from_numpy(a).to(cuda) for a in want[:2]), sd, cd,
                           *((torch.from_numpy(a).to(cuda) for a in want[2:4]) if qjl else ()))
    _bits_eq(y.cpu().numpy(), want_y)


@pytest.mark.parametrize("d", [16, 64, 128, 256])
def test_fwht_bitexact(cuda, d):
    ops = _ops()
    x = torch.randn(1001, d) * 3
    got = ops.fwht(x.to(cuda)).cpu().numpy()
    assert np.array_equal(got, ref.hadamard_np(x.numpy()))
    assert np.array_equal(got, ref.hadamard(x).numpy())


def test_vq_prepare_bitexact(cuda):
    ops = _ops()
    g = torch.Generator().manual_seed(3)
    B, G, T, D, start, end = 2, 8, 300, 128, 4, 236
    v = torch.randn(B, G, T, D, generator=g).half()
    v[:, :, :, 7] *= 8
    vm = v[:, :, start:end, :].float().reshape(B * G, end - start, D)
    rot = ref.hadamard(vm)
    ch = rot.abs().amax(dim=1).clamp(min=1e-8)
    want = (rot / ch.unsqueeze(1)).reshape(-1, 4)
    x, ch32, ch16 = ops.vq_prepare(v.to(cuda)[:, :, start:end, :].reshape(B * G, end - start, D))
    assert np.array_equal(ch32.cpu().numpy(), ch.numpy())
    assert np.array_equal(ch16.cpu().numpy().view(np.uint16), ch.half().numpy().view(np.uint16))
    assert np.array_equal(x.cpu().numpy().view(np.uint32), want.numpy().view(np.uint32))


@pytest.mark.parametrize("D", [64, 128, 256])
def test_vq_prepare_bits_at_the_edges(cuda, D):
    """shard_vq_prepare's rows and channel scales bit for bit (signed zeros
    included) against the reference's hadamard + division, per head size, on
    heads built to reach the divisions' edges: an all-zero head (scales
    clamped to 1e-8), a head of negative zeros, rows at +-65504, fp16
    subnormals, and a head holding an infinity (infinite scales: that head
    divides with the IEEE sequence)."""
    ops = _ops()
    g = torch.Generator().manual_seed(30 + D)
    BG, T = 7, 257
    v = torch.randn(BG, T, D, generator=g).half()
    v[0, :, 5] *= 8
    v[1] = 0.0
    v[2] = -0.0
    v[3, 0, :] = 65504.0
    v[3, 1, :] = -65504.0
    v[4] = (v[4].float() * 1e-6).half()
    v[6, 3, 9] = float("inf")
    rot = ref.hadamard(v.float())
    ch = rot.abs().amax(dim=1).clamp(min=1e-8)
    with np.errstate(all="ignore"):
        want = (rot / ch.unsqueeze(1)).reshape(BG, -1).numpy()
    x, ch32, _ = ops.vq_prepare(v.to(cuda))
    assert np.array_equal(ch32.cpu().numpy().view(np.uint32), ch.numpy().view(np.uint32))
    got = x.cpu().numpy().reshape(BG, -1)
    assert np.array_equal(got[:6].view(np.uint32), want[:6].view(np.uint32))
    nan = np.isnan(want[6])
    assert np.array_equal(np.isnan(got[6]), nan)
    assert np.array_equal(got[6][~nan].view(np.uint32), want[6][~nan].view(np.uint32))


def test_vq_assign_bitexact(cuda):
    ops = _ops()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(300001, 4, generator=g)
    c = torch.randn(256, 4, generator=g)
    got = ops.vq_assign(x.to(cuda), c.to(cuda)).cpu().numpy()
    want = ref.vq_assign_direct(x.numpy(), c.numpy())
    assert np.array_equal(got, want)
    mism = int((got != ref.vq_assign_cdist(x, c).numpy()).sum())
    assert mism == 0, f"{mism} rows differ from torch.cdist argmin"


def _vq_hard_rows(c, g):
    """Rows that stress the MFMA screen's certification: midpoints of centroid
    pairs (near and exact fp32 ties), rows on and near centroids, zero rows,
    rows far outside the screen's scale range, and non-finite rows."""
    k = c.shape[0]
    a = torch.randint(0, k, (6000,), generator=g)
    b = torch.randint(0, k, (6000,), generator=g)
    mid = 0.5 * (c[a] + c[b])
    nan, inf = float("nan"), float("inf")
    special = torch.tensor([[nan, 0, 0, 0], [inf, 0, 0, 0], [-inf, 1, 2, 3], [1e30, 0, 0, 0],
                            [0, 0, 0, 0], [1e-40, 0, 0, 0], [-0.0, 0, 0, 0]])
    return torch.cat([torch.randn(9000, 4, generator=g), mid,
                      mid + 1e-7 * torch.randn(6000, 4, generator=g),
                      c[a] + 1e-6 * torch.randn(6000, 4, generator=g), c[a[:500]],
                      torch.zeros(100, 4), 1e20 * torch.randn(500, 4, generator=g),
                      1e-25 * torch.randn(500, 4, generator=g), special])


@pytest.mark.parametrize("k", [32, 96, 160, 256])
def test_vq_assign_hard_rows_bitexact(cuda, k):
    """The MFMA-screened assignment (d = 4, k = 32 NB) against the sequential
    direct-distance oracle on rows built to defeat the screen, with duplicate
    and zero centroids (exact ties: first index wins)."""
    ops = _ops()
    g = torch.Generator().manual_seed(1000 + k)
    c = torch.randn(k, 4, generator=g)
    c[3] = c[5]
    c[7] = 0.0
    c[k - 1] = c[0] * (1 + 2 ** -20)
    x = _vq_hard_rows(c, g)
    x = x[torch.randperm(x.shape[0], generator=g)][: x.shape[0] - 13]  # ragged tail
    got = ops.vq_assign(x.to(cuda), c.to(cuda)).cpu().numpy()
    with np.errstate(all="ignore"):
        want = ref.vq_assign_direct(x.numpy(), c.numpy())
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: got {got[bad[:5]]} want {want[bad[:5]]}"


@pytest.mark.parametrize("case", ["nan_centroid", "tiny_centroids", "huge_centroids"])
def test_vq_assign_out_of_range_centroids_bitexact(cuda, case):
    """Centroid sets the screen must not certify (non-finite, or far outside its
    scale range): every row falls back to the reference's distances."""
    ops = _ops()
    g = torch.Generator().manual_seed(77)
    c = torch.randn(256, 4, generator=g)
    if case == "nan_centroid":
        c[9] = float("nan")
        c[10, 2] = float("inf")
    elif case == "tiny_centroids":
        c = c * 1e-30
    else:
        c = c * 1e25
    x = torch.randn(4099, 4, generator=g) * (1e-30 if case == "tiny_centroids" else 1.0)
    got = ops.vq_assign(x.to(cuda), c.to(cuda)).cpu().numpy()
    with np.errstate(all="ignore"):
        want = ref.vq_assign_direct(x.numpy(), c.numpy())
    assert np.array_equal(got, want)


def _normalized_rows(n, g):
    """Rows shaped like shard_vq_prepare's output: in [-1, 1], most mass near
    0 (Gaussian / 4), the channel maxima at exactly +-1."""
    x = (0.25 * torch.randn(n, 4, generator=g)).clamp(-1.0, 1.0)
    x[:64] = torch.where(torch.rand(64, 4, generator=g) < 0.5, -1.0, 1.0)
    return x


def _table_rows(c, g):
    """Rows for the candidate table: normalized rows, hard rows (midpoints and
    near ties of centroid pairs, rows on centroids, zero rows) squeezed into
    the box, rows on cell boundaries and box faces, just outside the box, far
    outside it, and non-finite rows."""
    k = c.shape[0]
    a = torch.randint(0, k, (4000,), generator=g)
    b = torch.randint(0, k, (4000,), generator=g)
    mid = 0.5 * (c[a] + c[b])
    edges = torch.linspace(-1.0, 1.0, 21)[torch.randint(0, 21, (4000, 4), generator=g)]
    nan, inf = float("nan"), float("inf")
    special = torch.tensor([[nan, 0, 0, 0], [inf, 0, 0, 0], [-inf, 0.5, 0, 0], [1e30, 0, 0, 0],
                            [1.0000001, 0, 0, 0], [-1.0000001, 0.3, 0.2, 0.1], [1.001, 1, 1, 1],
                            [0, 0, 0, 0], [1e-40, 0, 0, 0], [-0.0, 0, 0, 0], [1, 1, 1, 1],
                            [-1, -1, -1, -1]])
    return torch.cat([_normalized_rows(40000, g), mid,
                      mid + 1e-7 * torch.randn(4000, 4, generator=g),
                      c[a] + 1e-6 * torch.randn(4000, 4, generator=g), c[a[:300]],
                      edges, edges + 1e-7 * torch.randn(4000, 4, generator=g),
                      torch.zeros(50, 4), 3.0 * torch.randn(500, 4, generator=g), special])


def _table_case(k, g):
    """A codebook drawn from normalized rows with duplicate, zero and
    nearly-equal centroids (exact ties: first index wins)."""
    c = _normalized_rows(4 * k, g)[64 + torch.randperm(4 * k - 64, generator=g)[:k]].clone()
    c[3] = c[5]
    c[7] = 0.0
    c[k - 1] = c[0] * (1 + 2 ** -20)
    return c


@pytest.mark.parametrize("k,nbins", [(256, 20), (256, 32), (96, 8), (32, 1), (256, 3)])
def test_vq_assign_table_bitexact(cuda, k, nbins):
    """Nearest centroid through the candidate table (most rows decided from
    their cell's list, the rest by the all-centroid kernel) against the
    sequential direct-distance oracle, on rows built to sit on cell boundaries,
    box faces, near ties and outside the box."""
    ops = _ops()
    g = torch.Generator().manual_seed(4000 + 7 * k + nbins)
    c = _table_case(k, g)
    x = _table_rows(c, g)
    x = x[torch.randperm(x.shape[0], generator=g)][: x.shape[0] - 13]  # ragged tail
    table = ops.VqTable(c.to(cuda), nbins=nbins)
    got = ops.vq_assign_table(x.to(cuda), table).cpu().numpy()
    with np.errstate(all="ignore"):
        want = ref.vq_assign_direct(x.numpy(), c.numpy())
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: got {got[bad[:5]]} want {want[bad[:5]]}"
    # and the same as the all-centroid kernel
    assert np.array_equal(got, ops.vq_assign(x.to(cuda), c.to(cuda)).cpu().numpy())


@pytest.mark.parametrize("B,G,T,nbins", [(2, 8, 772, 16), (1, 3, 325, 3)])
def test_vq_encode_table_equals_prepare_then_assign(cuda, B, G, T, nbins):
    """The fused V encoder (subvectors formed from V in registers, assigned
    through the table, never written out) against shard_vq_prepare followed
    by the table assignment, bit for bit, on a slice of the sequence (a row
    stride past the slice), with outlier channels, a head at +-65504, an
    all-zero head, a head holding an infinity (the IEEE division path), an odd
    token count (a wave straddling the end) and, at 3 cells per dim, most
    rows left to the all-centroid kernel (rows passed with their values)."""
    ops = _ops()
    g = torch.Generator().manual_seed(B * 1000 + T)
    v = torch.randn(B, G, T, 128, generator=g).half()
    v[..., 9] *= 8
    v[0, 1, 7, :] = 65504.0
    v[0, 1, 8, :] = -65504.0
    v[0, 2] = 0.0
    if G > 3:
        v[0, 3, 11, 40] = float("inf")
    start, end = 4, T - 64
    vs = v.to(cuda)[:, :, start:end, :].reshape(B * G, end - start, 128)
    x, ch32, ch16 = ops.vq_prepare(vs)
    s32, s16, rcp = ops.vq_scales(vs)
    assert np.array_equal(s32.cpu().numpy().view(np.uint32), ch32.cpu().numpy().view(np.uint32))
    assert np.array_equal(s16.cpu().numpy().view(np.uint16), ch16.cpu().numpy().view(np.uint16))
    assert torch.equal(rcp.cpu(), 1.0 / ch32.cpu())
    gsel = torch.Generator().manual_seed(7)
    finite = torch.isfinite(x).all(1)
    pool = x[finite]
    cb = pool[torch.randperm(pool.shape[0], generator=gsel)[:256].to(cuda)].contiguous()
    table = ops.VqTable(cb, nbins=nbins)
    want = ops.vq_assign_table(x, table)
    got = ops.vq_encode_table(vs, s32, rcp, table)
    assert torch.equal(got, want), int((got != want).sum())


def _read_table(table):
    """(counts (cells,), lists (cells, 32)) of a built table."""
    raw = table.table.cpu().numpy()
    cells = table.nbins ** 4
    counts = raw[64:64 + cells]
    off = 64 + ((cells + 15) & ~15)
    lists = raw[off:off + 32 * cells].reshape(cells, 32)
    return counts, lists


def test_vq_table_lists_every_nearest_centroid(cuda):
    """The table's own contract, cell by cell: counts within 1..32 (255 marks a
    cell whose rows take the other path), lists ascending and padded with
    their last entry, and for sampled rows of each sampled cell (its corners,
    its centre, random interior points) the oracle's nearest centroid is
    listed."""
    ops = _ops()
    g = torch.Generator().manual_seed(31)
    k, nbins = 256, 12
    c = _table_case(k, g)
    table = ops.VqTable(c.to(cuda), nbins=nbins)
    counts, lists = _read_table(table)
    listed = counts != 255
    assert listed.mean() > 0.99
    assert counts[listed].min() >= 1 and counts[listed].max() <= 32
    w = 2.0 / nbins
    cells = torch.randperm(nbins ** 4, generator=g)[:3000].numpy()
    rows, owner = [], []
    for cell in cells:
        ijk = np.array([(cell // nbins ** (3 - j)) % nbins for j in range(4)])
        lo = -1.0 + ijk * w
        corners = lo + w * np.array([[(m >> j) & 1 for j in range(4)] for m in range(16)])
        inner = lo + w * torch.rand(8, 4, generator=g).numpy()
        pts = np.concatenate([corners, inner, (lo + 0.5 * w)[None]]).astype(np.float32)
        rows.append(pts)
        owner += [cell] * len(pts)
    rows = np.concatenate(rows)
    owner = np.array(owner)
    want = ref.vq_assign_direct(rows, c.numpy())
    for cell in cells:
        n = counts[cell]
        if n == 255:
            continue
        lst = lists[cell]
        assert np.all(np.diff(lst[:n].astype(int)) > 0), "list not ascending"
        assert np.all(lst[n:] == lst[n - 1]), "padding is not the last candidate"
        assert np.all(np.isin(want[owner == cell], lst[:n])), f"cell {cell} misses a nearest centroid"


@pytest.mark.parametrize("case", ["nan_centroid", "huge_centroids", "other_box"])
def test_vq_assign_table_undecidable_tables_bitexact(cuda, case):
    """Tables that decide nothing (a non-finite centroid, centroids above 2^32,
    or a call whose box differs from the build's): every row takes the
    all-centroid path and the result is still the oracle's."""
    ops = _ops()
    g = torch.Generator().manual_seed(78)
    c = _table_case(256, g)
    if case == "nan_centroid":
        c[9] = float("nan")
        c[10, 2] = float("inf")
    elif case == "huge_centroids":
        c[11] = 1e12
    x = _normalized_rows(9000, g)
    table = ops.VqTable(c.to(cuda))
    if case == "other_box":
        table.hi = 2.0  # a table built for [-1, 1] used as if for [-1, 2]
    lib = __import__("shard_amd._lib", fromlist=["load"]).load()
    ws = torch.zeros(lib.shard_vq_assign_table_workspace(x.shape[0]), dtype=torch.uint8, device=cuda)
    got = ops.vq_assign_table(x.to(cuda), table, ws=ws).cpu().numpy()
    with np.errstate(all="ignore"):
        want = ref.vq_assign_direct(x.numpy(), c.numpy())
    assert np.array_equal(got, want)
    assert ops.vq_undecided_rows(ws, x.shape[0]) == x.shape[0]  # every row took the other path


def test_vq_assign_table_decides_normalized_rows_itself(cuda):
    """On normalized rows (shard_vq_prepare's range) with a codebook drawn
    from them, the table decides almost every row (the undecided count is
    the workspace's first word)."""
    ops = _ops()
    g = torch.Generator().manual_seed(79)
    c = _table_case(256, g)
    x = _normalized_rows(200000, g)
    table = ops.VqTable(c.to(cuda))
    lib = __import__("shard_amd._lib", fromlist=["load"]).load()
    ws = torch.zeros(lib.shard_vq_assign_table_workspace(x.shape[0]), dtype=torch.uint8, device=cuda)
    got = ops.vq_assign_table(x.to(cuda), table, ws=ws).cpu().numpy()
    assert np.array_equal(got, ref.vq_assign_direct(x.numpy(), c.numpy()))
    undecided = ops.vq_undecided_rows(ws, x.shape[0])
    assert undecided < 0.001 * x.shape[0], undecided


def test_kmeans_through_the_table_equals_the_all_centroid_path(cuda, monkeypatch):
    """k-means with the per-iteration candidate table (taken from
    VQ_TABLE_MIN_ROWS rows on) gives the same centroids and indices as with
    the all-centroid assignment, on normalized rows from shard_vq_prepare."""
    ops = _ops()
    g = torch.Generator().manual_seed(5)
    v = torch.randn(2, 8, 700, 128, generator=g).half()
    v[..., 3] *= 8
    x, _, _ = ops.vq_prepare(v.to(cuda).reshape(16, 700, 128))
    c1, i1 = ops.kmeans(x, 256, n_iter=6)
    calls = []
    real = ops.vq_assign_table
    monkeypatch.setattr(ops, "VQ_TABLE_MIN_ROWS", 0)
    monkeypatch.setattr(ops, "vq_assign_table", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    c2, i2 = ops.kmeans(x, 256, n_iter=6)
    assert len(calls) == 6
    assert torch.equal(c1, c2) and torch.equal(i1, i2)


@pytest.mark.parametrize("n,k,d,assign", [(70000, 256, 4, "nearest"), (9000, 1000, 8, "random"),
                                          (4097, 3, 2, "random"), (130, 1, 1, "random"),
                                          (200000, 64, 4, "skewed")])
def test_kmeans_update_bitexact(cuda, n, k, d, assign):
    """The update against torch CPU index_add_ (the reference's order:
    cache.py:30-33): rows summed per centroid in increasing row order, across
    sort blocks of 4096 rows, partial blocks and rounds, 1 to 1000 centroids
    (a centroid with most rows, one without rows) and rows of 1 to 8 values."""
    ops = _ops()
    g = torch.Generator().manual_seed(n + k)
    x = torch.randn(n, d, generator=g)
    c = x[torch.randperm(n, generator=g)[:k]].clone()
    if assign == "nearest":
        c[17] = 100.0  # an empty cluster keeps its centroid
        idx = torch.from_numpy(ref.vq_assign_direct(x.numpy(), c.numpy()))
    elif assign == "skewed":
        idx = torch.where(torch.rand(n, generator=g) < 0.7, torch.zeros(n, dtype=torch.int64),
                          torch.randint(0, k - 1, (n,), generator=g))
    else:
        idx = torch.randint(0, max(k - 1, 1), (n,), generator=g)  # the last centroid empty (k > 1)
    new = torch.zeros_like(c)
    cnt = torch.zeros(k)
    new.index_add_(0, idx, x)
    cnt.index_add_(0, idx, torch.ones(n))
    nz = cnt > 0
    new[nz] /= cnt[nz].unsqueeze(1)
    new[~nz] = c[~nz]
    got, maxd = ops.kmeans_update(x.to(cuda), idx.to(torch.int32).to(cuda), c.to(cuda))
    assert np.array_equal(got.cpu().numpy(), new.numpy())
    assert maxd.item() == (new - c).abs().max().item()


def test_kmeans_matches_reference_golden(cuda, golden):
    ops = _ops()
    gld = golden("kmeans.npz")
    cent, idx = ops.kmeans(torch.from_numpy(gld["data"]).to(cuda), int(gld["k"]), int(gld["n_iter"]),
                           int(gld["seed"]))
    assert np.array_equal(cent.cpu().numpy(), gld["centroids"])
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), gld["idx"])


@pytest.mark.parametrize("m,k,n", [(1000, 1024, 192), (4099, 1024, 64), (257, 512, 256), (31, 64, 32),
                                   (700, 1024, 320), (129, 256, 544)])  # wider: one launch per 256 columns
def test_pca_project_mfma(cuda, m, k, n):
    ops = _ops()
    g = torch.Generator().manual_seed(m)
    a = torch.randn(m, k, generator=g).half()
    bt = (torch.randn(n, k, generator=g) * 0.05).half()
    got = ops.pca_project(a.to(cuda), bt.to(cuda)).cpu().double()
    want = a.double() @ bt.double().T
    scale = (a.double().abs() @ bt.double().abs().T)
    assert float(((got - want).abs() / scale).max()) < 1e-5


@pytest.mark.parametrize("m,k,n", [(1980, 1024, 192), (4099, 1024, 64), (257, 512, 256), (31, 40, 32),
                                   (130, 1024, 96), (700, 1024, 320), (129, 256, 544)])
def test_pca_project_f32_mfma(cuda, m, k, n):
    """The fp32 projection (Cache.compress's GEMM) within fp32 summation error
    of the float64 product, including row tails, k past the last 32-chunk and
    column counts that leave a wave half idle."""
    ops = _ops()
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(m, k, generator=g)
    bt = torch.randn(n, k, generator=g) * 0.05
    got = ops.pca_project_f32(a.to(cuda), bt.to(cuda)).cpu().double()
    want = a.double() @ bt.double().T
    scale = a.double().abs() @ bt.double().abs().T
    err = float(((got - want).abs() / scale).max())
    print(f"pca_project_f32 m={m} k={k} n={n}: max rel err {err:.3e}", flush=True)
    assert err < 4e-7 * (k / 1024) ** 0.5 * 8


def test_k_prepare_f32(cuda):
    """The fp32 centred rows of (flat - mean) (cache.py:370-392): undo RoPE
    with fp32 phases, the mean subtracted in fp32, no fp16 rounding."""
    ops = _ops()
    g = torch.Generator().manual_seed(3)
    B, G, T, D, start, n_comp = 2, 8, 200, 128, 4, 132
    k = torch.randn(B, G, T, D, generator=g).half()
    inv = ref.default_inv_freq(500000.0, D)
    pos = torch.arange(start, start + n_comp)
    un = ref.undo_rope(k[:, :, start:start + n_comp].float(), pos, inv)
    flat = un.permute(0, 2, 1, 3).reshape(B * n_comp, G * D)
    mean = flat.mean(0)
    want = flat - mean
    got = ops.k_prepare(k.to(cuda), start, n_comp, inv.to(cuda), mean.to(cuda),
                        out_dtype=torch.float32).cpu()
    # sin/cos may differ by an ulp from torch's CPU ones
    assert float((got - want).abs().max()) <= 4e-7 * float(want.abs().max())


@pytest.mark.parametrize("B,G,T,start,n_comp,n", [(2, 8, 300, 4, 232, 192), (1, 8, 700, 4, 632, 64),
                                                    (3, 4, 200, 0, 200, 256),
                                                    # k chunk counts (2 per kv head) that are not
                                                    # a multiple of the key ring
                                                    (1, 2, 150, 4, 100, 96), (2, 6, 130, 0, 130, 128)])
def test_pca_project_rope_equals_prepare_then_project(cuda, B, G, T, start, n_comp, n):
    """The fused front end (undo RoPE in the A loads, permuted k order) computes
    the same fp16 operand as shard_k_prepare with a zero mean, so it matches
    k_prepare + pca_project to fp32 summation order; with a mean, the bias
    mean . basis stands for the centring (fp64 check)."""
    ops = _ops()
    g = torch.Generator().manual_seed(T + n)
    k = (torch.randn(B, G, T, 128, generator=g) * 2).half()
    bt = (torch.randn(n, G * 128, generator=g) * 0.03).half()
    inv = ref.default_inv_freq(500000.0, 128)
    kd, btd, invd = k.to(cuda), bt.to(cuda), inv.to(cuda)
    ph = ops.rope_phases(start, n_comp, invd)
    zero = torch.zeros(G * 128, device=cuda)
    want = ops.pca_project(ops.k_prepare(kd, start, n_comp, invd, zero), btd).cpu().double()
    btp = ops.rope_basis(btd)
    got = ops.pca_project_rope(kd, start, n_comp, ph, btp).cpu().double()
    a16 = ops.k_prepare(kd, start, n_comp, invd, zero).cpu().double()
    exact = a16 @ bt.double().T              # the common fp16 operand, summed in fp64
    scale = a16.abs() @ bt.double().abs().T
    err = float(((got - exact).abs() / scale).max())
    err_u = float(((want - exact).abs() / scale).max())
    print(f"pca_project_rope B={B} G={G} n_comp={n_comp} n={n}: max rel err {err:.3e} "
          f"(unfused {err_u:.3e})", flush=True)
    assert err < 1e-6 and err_u < 1e-6
    # a mean: fp16(undo(k)) . B - mean . B against fp64 (undo(k) - mean) . B
    mean = torch.randn(G * 128, generator=g) * 0.1
    bias = (mean.double() @ bt.double().T).float()
    got_m = ops.pca_project_rope(kd, start, n_comp, ph, btp, bias=bias.to(cuda)).cpu().double()
    un = ref.undo_rope(k[:, :, start:start + n_comp].float(), torch.arange(start, start + n_comp), inv)
    x = un.permute(0, 2, 1, 3).reshape(B * n_comp, G * 128).double() - mean.double()
    want_m = x @ bt.double().T
    err_m = float(((got_m - want_m).abs() / (x.abs() @ bt.double().abs().T)).max())
    assert err_m < 2e-3


def test_k_prepare(cuda):
    ops = _ops()
    g = torch.Generator().manual_seed(2)
    B, G, T, D, start, n_comp = 2, 8, 200, 128, 4, 132
    k = torch.randn(B, G, T, D, generator=g).half()
    inv = ref.default_inv_freq(500000.0, D)
    pos = torch.arange(start, start + n_comp)
    un = ref.undo_rope(k[:, :, start:start + n_comp].float(), pos, inv)
    flat = un.permute(0, 2, 1, 3).reshape(B * n_comp, G * D)
    mean = flat.mean(0)
    want = (flat - mean).half().float()
    got = ops.k_prepare(k.to(cuda), start, n_comp, inv.to(cuda), mean.to(cuda)).cpu().float()
    # sin/cos may differ by an ulp from torch's CPU ones: allow one fp16 ulp
    assert float((got - want).abs().max()) <= 2e-3 * float(want.abs().max())


@pytest.mark.parametrize("B,H,G,hd,bits,qjl,shared", [(16, 32, 8, 128, 8, False, True),
                                                      (4, 32, 8, 128, 8, False, False),
                                                      (2, 32, 8, 128, 4, True, False),
                                                      (1, 8, 2, 256, 8, False, False),
                                                      (3, 32, 8, 64, 8, False, False),
                                                      (2, 8, 2, 64, 4, True, True)])
def test_rope_stream_append_bitexact(cuda, B, H, G, hd, bits, qjl, shared):
    """The decode-step front end (one launch) against its two reference steps:
    transformers' apply_rotary_pos_emb on fp16 CPU tensors (the library routine
    the reference's patched forward calls, attention.py:376) for q and k, then
    the stream quantizer oracle on the rotated k and on v (cache.py:207-215).
    shared: one cos/sin row for the whole batch, as the model passes it when
    every sequence is at the same position."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    ops = _ops()
    g = torch.Generator().manual_seed(B * 100 + hd + bits)
    q = (torch.randn(B, H, 1, hd, generator=g) * 3).half()
    k = (torch.randn(B, G, 1, hd, generator=g) * 3).half()
    v = torch.randn(B, G, 1, hd, generator=g).half()
    pos = torch.randint(0, 40000, (1 if shared else B, 1), generator=g)
    inv = torch.as_tensor(ref.default_inv_freq(500000.0, hd), dtype=torch.float32)
    freqs = pos[..., None].float() * inv[None, None, :]
    emb = torch.cat([freqs, freqs], -1)
    cos, sin = emb.cos().half(), emb.sin().half()          # (B, 1, hd), as the model passes them
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos, sin)
    cb = ref.lloyd_max_codebook(hd, bits)
    signs = ref.stream_signs(3, hd)
    wk = ref.quantize_stream_token(k_ref.reshape(B, G, hd).numpy(), signs, cb, qjl=qjl)
    wv = ref.quantize_stream_token(v.reshape(B, G, hd).numpy(), signs, cb, qjl=qjl)

    dev = lambda t: t.to(cuda).contiguous()
    out = {n: torch.empty(B, G, hd, dtype=torch.uint8, device=cuda) for n in ("ki", "vi", "ks", "vs")}
    out.update({n: torch.empty(B, G, dtype=torch.float16, device=cuda) for n in ("kn", "vn", "kc", "vc")})
    out.update({n: torch.empty(B, G, hd, dtype=torch.float16, device=cuda) for n in ("kd", "vd")})
    q_out = torch.empty(B, H, hd, dtype=torch.float16, device=cuda)
    p = lambda n: out[n].data_ptr()
    qj = (p("ks"), p("kc"), p("vs"), p("vc")) if qjl else (None, None, None, None)
    ops.rope_stream_append_at(dev(q.reshape(B, H, hd)), dev(k.reshape(B, G, hd)),
                              dev(v.reshape(B, G, hd)), dev(cos.reshape(-1, hd)),
                              dev(sin.reshape(-1, hd)), dev(torch.from_numpy(signs)),
                              dev(torch.from_numpy(cb)), q_out, p("ki"), p("kn"), p("kd"),
                              p("vi"), p("vn"), p("vd"), *qj)
    torch.cuda.synchronize()
    _bits_eq(q_out.cpu().numpy(), q_ref.reshape(B, H, hd).numpy())
    for want, (i, n, s, c, d) in ((wk, ("ki", "kn", "ks", "kc", "kd")),
                                  (wv, ("vi", "vn", "vs", "vc", "vd"))):
        assert np.array_equal(out[i].cpu().numpy(), want[0])
        _bits_eq(out[n].cpu().numpy(), want[1])
        if qjl:
            assert np.array_equal(out[s].cpu().numpy(), want[2])
            _bits_eq(out[c].cpu().numpy(), want[3])
        want_y = ref.dequantize_stream_token(want[0], want[1], signs, cb,
                                             *(want[2:4] if qjl else (None, None)))
        _bits_eq(out[d].cpu().numpy(), want_y)


@pytest.mark.parametrize("bits,qjl", [(8, False), (3, True)])
def test_stream_quant_kv_rows_bitexact(cuda, bits, qjl):
    """One launch for a token's K and V (shard_stream_quant_kv) writing into row
    s of (cap, B, G, D) buffers by address: the row equals the oracle's codes,
    norms, QJL terms and fp16 rows, and the other rows are untouched."""
    ops = _ops()
    B, G, D, cap, s = 3, 8, 128, 5, 2
    g = torch.Generator().manual_seed(bits)
    k = (torch.randn(B, G, D, generator=g) * 2).half()
    v = torch.randn(B, G, D, generator=g).half()
    cb = ref.lloyd_max_codebook(D, bits)
    signs = ref.stream_signs(7, D)
    wk = ref.quantize_stream_token(k.numpy(), signs, cb, qjl=qjl)
    wv = ref.quantize_stream_token(v.numpy(), signs, cb, qjl=qjl)
    bufs = {n: torch.full((cap, B, G, D), 0x55, dtype=torch.uint8, device=cuda) for n in ("ki", "vi", "ks", "vs")}
    bufs.update({n: torch.full((cap, B, G), 7.0, dtype=torch.float16, device=cuda) for n in ("kn", "vn", "kc", "vc")})
    bufs.update({n: torch.full((cap, B, G, D), 7.0, dtype=torch.float16, device=cuda) for n in ("kd", "vd")})
    row = lambda n: bufs[n][s].data_ptr()
    qj = (row("ks"), row("kc"), row("vs"), row("vc")) if qjl else (None, None, None, None)
    ops.stream_quant_kv_at(k.to(cuda), v.to(cuda), torch.from_numpy(signs).to(cuda),
                           torch.from_numpy(cb).to(cuda), row("ki"), row("kn"), row("kd"),
                           row("vi"), row("vn"), row("vd"), *qj)
    torch.cuda.synchronize()
    for want, (i, n, sg, c, d) in ((wk, ("ki", "kn", "ks", "kc", "kd")),
                                   (wv, ("vi", "vn", "vs", "vc", "vd"))):
        assert np.array_equal(bufs[i][s].cpu().numpy(), want[0])
        _bits_eq(bufs[n][s].cpu().numpy(), want[1])
        if qjl:
            assert np.array_equal(bufs[sg][s].cpu().numpy(), want[2])
            _bits_eq(bufs[c][s].cpu().numpy(), want[3])
        want_y = ref.dequantize_stream_token(want[0], want[1], signs, cb,
                                             *(want[2:4] if qjl else (None, None)))
        _bits_eq(bufs[d][s].cpu().numpy(), want_y)
        for other in (0, 1, 3, 4):  # rows other than s keep their fill
            assert bool((bufs[i][other] == 0x55).all()) and bool((bufs[d][other] == 7.0).all())


def test_prefill_kernels_at_config4_layer_size(cuda):
    """One layer of the prefill workload (batch 4 x 8192 tokens, 8 kv heads): the V
    front end and the int4 chain bit-exact, the projection within fp32 summation
    error, at the sizes whose multi-block reductions and grid-stride loops the
    small cases above do not reach."""
    ops = _ops()
    g = torch.Generator().manual_seed(4)
    B, G, T, D = 4, 8, 8192, 128
    v = torch.randn(B, G, T, D, generator=g).half()
    v[:, :, :, 3] *= 8
    x, ch32, _ = ops.vq_prepare(v.to(cuda).reshape(B * G, T, D))
    rot = ref.hadamard(v.float().reshape(B * G, T, D))
    ch = rot.abs().amax(dim=1).clamp(min=1e-8)
    assert np.array_equal(ch32.cpu().numpy(), ch.numpy())
    assert np.array_equal(x.cpu().numpy().view(np.uint32),
                          (rot / ch.unsqueeze(1)).reshape(-1, 4).numpy().view(np.uint32))
    del rot
    # the layer's nearest-centroid stage at full size: its 8.4M subvectors
    # against a seeded codebook drawn from them, bit-exact with the C oracle
    from oracle import cref
    if cref.load() is None:
        cref.build()
    gsel = torch.Generator().manual_seed(42)
    xc = x.cpu()
    codebook = xc[torch.randperm(xc.shape[0], generator=gsel)[:256]].contiguous()
    print(f"[config4 layer] vq_assign on {xc.shape[0]} subvectors", flush=True)
    idx = ops.vq_assign(x, codebook.to(cuda)).cpu().numpy().astype(np.int64)
    want_idx = cref.vq_assign_direct(xc.numpy(), codebook.numpy())
    assert np.array_equal(idx, want_idx), int((idx != want_idx).sum())
    print(f"[config4 layer] vq_assign_table on {xc.shape[0]} subvectors", flush=True)
    table = ops.VqTable(codebook.to(cuda))
    tidx = ops.vq_assign_table(x, table).cpu().numpy().astype(np.int64)
    assert np.array_equal(tidx, want_idx), int((tidx != want_idx).sum())
    print(f"[config4 layer] vq_encode_table on {xc.shape[0]} subvectors", flush=True)
    vr = v.to(cuda).reshape(B * G, T, D)
    s32, _, rcp = ops.vq_scales(vr)
    eidx = ops.vq_encode_table(vr, s32, rcp, table).cpu().numpy().astype(np.int64)
    assert np.array_equal(eidx, want_idx), int((eidx != want_idx).sum())
    del x, xc

    # the K front end at full size: undo RoPE and centring into the fp16 operand
    kk = (torch.randn(B, G, T, D, generator=g) * 2).half()
    inv = ref.default_inv_freq(500000.0, D)
    un = ref.undo_rope(kk.float(), torch.arange(T), inv).permute(0, 2, 1, 3).reshape(B * T, G * D)
    mean = un.mean(0)
    want_kp = (un - mean).half().float()
    kp = ops.k_prepare(kk.to(cuda), 0, T, inv.to(cuda), mean.to(cuda)).cpu().float()
    # sin/cos of phases up to 8191 rad may differ by a few fp32 ulps from torch's
    # CPU ones: |k| <= 12 gives an fp32 difference below 1e-5 before the fp16
    # rounding, so the operands agree to one fp16 ulp plus that
    ulp = torch.where(want_kp.abs() < 6.1e-5, torch.full_like(want_kp, 2.0 ** -24),
                      2.0 ** (torch.floor(torch.log2(want_kp.abs().clamp(min=6.1e-5))) - 10))
    err = (kp - want_kp).abs()
    print(f"[config4 layer] k_prepare: {int((err > 0).sum())} of {err.numel()} operands differ, "
          f"max {float(err.max()):.3e}", flush=True)
    assert bool((err <= ulp + 1e-5).all())
    del kk, un, kp, want_kp

    m, k, n = B * T, G * D, 192
    a = (torch.randn(m, k, generator=g) * 0.5).half()
    bt = (torch.randn(n, k, generator=g) * 0.03).half()
    proj = ops.pca_project(a.to(cuda), bt.to(cuda))
    want = a.double() @ bt.double().T
    scale = a.double().abs() @ bt.double().abs().T
    assert float(((proj.cpu().double() - want).abs() / scale).max()) < 1e-5

    p32 = proj.cpu().numpy()
    alloc = [4] * n
    chain = ref.k_code_chain(p32, alloc)
    got = ops.int4_quant_pack(proj, torch.tensor(alloc, dtype=torch.int32))
    assert np.array_equal(got["packed"].cpu().numpy(), chain["packed"])
    assert np.array_equal(got["coeff_scale"].cpu().numpy(), chain["coeff_scale"])


@pytest.mark.parametrize("qjl", [False, True])
def test_rope_stream_append_dev_row(cuda, qjl):
    """shard_rope_stream_append_dev: the token goes to the buffers' row
    row_dev[0] (read on the device), bit-identical to shard_rope_stream_append
    writing that row by address; every other row is untouched, and a row at or
    past row_cap writes no stream row (q after RoPE is still written)."""
    ops = _ops()
    B, H, G, hd, cap = 3, 8, 2, 128, 6
    g = torch.Generator().manual_seed(71)
    q = (torch.randn(B, H, hd, generator=g) * 3).half().to(cuda)
    k = (torch.randn(B, G, hd, generator=g) * 3).half().to(cuda)
    v = torch.randn(B, G, hd, generator=g).half().to(cuda)
    inv = torch.as_tensor(ref.default_inv_freq(500000.0, hd), dtype=torch.float32)
    emb = torch.cat([inv * 777.0, inv * 777.0])[None]
    cos, sin = emb.cos().half().to(cuda), emb.sin().half().to(cuda)
    signs = torch.from_numpy(ref.stream_signs(4, hd)).to(cuda)
    cb = torch.from_numpy(ref.lloyd_max_codebook(hd, 8)).to(cuda)

    def buffers():
        torch.manual_seed(5)
        u8 = lambda: torch.randint(0, 256, (cap, B, G, hd), dtype=torch.uint8).to(cuda)
        f16 = lambda *s: torch.randn(cap, B, G, *s).half().to(cuda)
        return {"ki": u8(), "vi": u8(), "ks": u8(), "vs": u8(), "kn": f16(), "vn": f16(),
                "kc": f16(), "vc": f16(), "kd": f16(hd), "vd": f16(hd)}

    order = ("ki", "kn", "kd", "vi", "vn", "vd")
    qorder = ("ks", "kc", "vs", "vc")
    for row in (0, 4, cap):
        want, got = buffers(), buffers()
        q_want = torch.empty(B, H, hd, dtype=torch.float16, device=cuda)
        q_got = torch.empty_like(q_want)
        r = min(row, cap - 1)
        if row < cap:
            at = lambda n: want[n][r].data_ptr()
            ops.rope_stream_append_at(q, k, v, cos, sin, signs, cb, q_want, *(at(n) for n in order),
                                      *((at(n) for n in qorder) if qjl else (None,) * 4))
        else:
            ops.rope_stream_append_at(q, k, v, cos, sin, signs, cb, q_want,
                                      *(want[n][r].data_ptr() for n in order),
                                      *((want[n][r].data_ptr() for n in qorder) if qjl else (None,) * 4))
            want = buffers()  # a row past the buffers: nothing is written
        row_dev = torch.tensor([row], dtype=torch.int32, device=cuda)
        base = lambda n: got[n].data_ptr()
        ops.rope_stream_append_at(q, k, v, cos, sin, signs, cb, q_got, *(base(n) for n in order),
                                  *((base(n) for n in qorder) if qjl else (None,) * 4),
                                  row_dev=row_dev, row_cap=cap)
        torch.cuda.synchronize()
        assert torch.equal(q_got, q_want), row
        for n in order + (qorder if qjl else ()):
            assert torch.equal(got[n], want[n]), (row, n)
