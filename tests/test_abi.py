"""The C ABI: libshard_hip.so loads on the CPU host and exports every entry
point include/shard_hip.h declares, with the struct layout the binding uses.
No kernel is launched here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            src = open(os.path.join(ROOT, "include", h)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names += re.findall(r"\b(shard_[a-z0-9_]+)\s*\(", src)
    return sorted(set(names))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("shard_decode_attn", "shard_stream_quant", "shard_pca_project",
                 "shard_int4_quant_pack", "shard_fwht", "shard_vq_assign", "shard_kv_reconstruct"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from shard_amd import _lib
    lib = _lib.load()
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(raw, name), f"{name} declared in shard_hip.h but not exported"
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert set(declared_functions()) <= bound, "binding misses a declared entry point"
    assert lib.shard_version().startswith(b"shard_hip")
    assert lib.shard_decode_args_size() == ctypes.sizeof(_lib.DecodeArgs)


def test_argument_errors_without_gpu_work():
    """Bad arguments are rejected on the host before any launch."""
    from shard_amd import _lib
    lib = _lib.load()
    assert lib.shard_fwht(None, None, 10, 128, None) == -1
    assert lib.shard_pca_project(None, 1, 16, 16, None, 32, None, 32, None) == -1
    assert lib.shard_decode_attn(None, None, 0, None) == -1
    args = _lib.DecodeArgs()
    assert lib.shard_decode_attn_workspace(ctypes.byref(args)) == 0
    assert lib.shard_decode_attn_noalloc(None, None) == -1
    assert lib.shard_decode_attn_noalloc(ctypes.byref(args), None) == -1


def test_vq_table_sizes_and_argument_checks():
    """The candidate-table entry points size and check on the host: the table
    is a 64-byte header, a count byte per cell (padded to 16) and 32 list
    bytes per cell; unsupported k, an empty or far-off-centre box and a short
    table are refused before any launch (placeholder pointers, never used)."""
    from shard_amd import _lib
    lib = _lib.load()
    assert lib.shard_vq_table_bytes(256, 20) == 64 + 160000 + 32 * 160000
    assert lib.shard_vq_table_bytes(32, 3) == 64 + 96 + 32 * 81
    assert lib.shard_vq_table_bytes(257, 20) == 0 and lib.shard_vq_table_bytes(256, 33) == 0
    big = 1 << 30
    p = ctypes.c_void_p(4096)
    assert lib.shard_vq_table_build(None, 256, -1.0, 1.0, 20, p, big, None) == -1
    assert lib.shard_vq_table_build(p, 100, -1.0, 1.0, 20, p, big, None) == -2
    assert lib.shard_vq_table_build(p, 256, 1.0, -1.0, 20, p, big, None) == -1
    assert lib.shard_vq_table_build(p, 256, 1000.0, 1001.0, 20, p, big, None) == -1
    assert lib.shard_vq_table_build(p, 256, -1.0, 1.0, 20, p, 100, None) == -4
    # 1000 rows: 16 groups of 64, 4 workgroups of 4 waves; per wave a count and
    # a region of 64 rows (with values: 16 more bytes per row)
    assert lib.shard_vq_assign_table_workspace(1000) == 16 * 4 + 16 * 64 * 4
    assert lib.shard_vq_encode_table_workspace(1000) == 16 * 4 + 16 * 64 * 4 + 16 * 64 * 16
    assert lib.shard_vq_assign_table_workspace(1 << 31) == 0
    assert lib.shard_vq_assign_table(p, 1000, p, 256, p, big, 20, -1.0, 1.0, p, p, 16, None) == -4
    assert lib.shard_vq_assign_table(p, 1000, p, 64, p, 100, 20, -1.0, 1.0, p, p, big, None) == -4
    # the V encoder: scales need V and an output; the fused encoder is head_dim 128 only
    assert lib.shard_vq_scales(None, 4, 100, 128, 12800, p, None, None, p, big, None) == -1
    assert lib.shard_vq_scales(p, 4, 100, 96, 9600, p, None, None, p, big, None) == -2
    assert lib.shard_vq_encode_table(p, 4, 100, 64, 6400, p, p, p, 256, p, big, 16, -1.0, 1.0,
                                     p, p, big, None) == -2
    assert lib.shard_vq_encode_table(p, 4, 100, 128, 12800, p, p, p, 256, p, big, 16, -1.0, 1.0,
                                     p, p, 16, None) == -4


def test_noalloc_refuses_calls_beyond_its_scratch_before_any_launch():
    """The size check of shard_decode_attn_noalloc runs on the host: with
    placeholder pointers (never dereferenced) and 375 forced splits the call
    needs 12.48 MB of partial rows, more than the 8 MiB scratch."""
    from shard_amd import _lib, ops
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim, a.rank, a.n_comp = 2, 32, 8, 128, 192, 4000
    for f in ("q", "inv_freq", "k_coeffs", "prep", "v_idx", "v_codebook", "v_ch", "out"):
        setattr(a, f, 16)
    a.n_splits, a.kernel = 375, 2
    need = lib.shard_decode_attn_workspace(ctypes.byref(a))
    assert need == 2 * 32 * 375 * (128 + 2) * 4 > ops.DECODE_NOALLOC_SCRATCH_BYTES
    assert lib.shard_decode_attn_noalloc(ctypes.byref(a), None) == -4
    assert str(need).encode() in lib.shard_last_error()


def test_cpu_tensor_is_rejected_loudly():
    import torch
    from shard_amd import ops
    with pytest.raises(ops.ShardHipUnavailable):
        ops.fwht(torch.zeros(4, 128))


def test_forced_row_split_beyond_its_extras_runs_token_tiled():
    """kernel = 1 (Cache._decode_kernel = 1) on a call with more than 2,048
    extra tokens (a long 8-bit stream; the reference appends without limit,
    cache.py:156-181) is planned on the token-tiled kernel instead of being
    refused: the workspace query (host only, no launch) gives the token-tiled
    plan's size, while a call within the row-split kernel's range keeps the
    row-split plan."""
    from shard_amd import _lib
    lib = _lib.load()

    def ws(kernel, n_stream):
        a = _lib.DecodeArgs()
        a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim, a.rank, a.n_comp = 1, 32, 8, 128, 192, 8124
        a.n_sink, a.n_win, a.n_stream, a.kernel = 4, 64, n_stream, kernel
        return lib.shard_decode_attn_workspace(ctypes.byref(a))

    assert ws(1, 3000) == ws(2, 3000) > 0
    assert ws(1, 100) != ws(2, 100)
    assert ws(1, 2048 - 68) != ws(2, 2048 - 68)   # the last count the row-split kernel takes
    assert ws(1, 2048 - 67) == ws(2, 2048 - 67)


def test_decode_shapes_and_sizes_on_the_host():
    """Up to 64 query heads per kv head at head_dim 128 (any count: groups of
    4, 3, 2 or 1 per workgroup), and head_dim 64 with an even kv head count
    (kv heads run in pairs as 128-dim heads, up to 32 query heads per kv head);
    the library agrees with ops.decode_supported; at head_dim 64 the workspace
    keeps 128-float partial rows and the prepare buffer holds one operand image
    per pair.  Host-only queries, no launch."""
    from shard_amd import _lib, ops
    lib = _lib.load()

    def supported(hd, n_q, n_kv, rank=192):
        a = _lib.DecodeArgs()
        a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim, a.rank, a.n_comp = 1, n_q, n_kv, hd, rank, 1000
        return lib.shard_decode_supported(ctypes.byref(a)) == 1

    for hd, n_q, n_kv, want in ((64, 32, 8, True), (64, 32, 4, True), (64, 8, 8, True),
                                (64, 4, 2, True), (64, 24, 4, True), (64, 12, 4, True),
                                (64, 9, 3, False), (64, 4, 8, False), (64, 64, 2, True),
                                (64, 66, 2, False), (64, 128, 2, False), (96, 32, 8, False),
                                (128, 24, 8, True), (128, 40, 8, True), (128, 56, 8, True),
                                (128, 512, 8, True), (128, 520, 8, False), (128, 12, 8, False)):
        assert supported(hd, n_q, n_kv) == want, (hd, n_q, n_kv)
        assert ops.decode_supported(hd, n_q, n_kv, 192) == want, (hd, n_q, n_kv)
    assert not supported(64, 32, 8, rank=100)   # rank must be padded to a multiple of 32
    a = _lib.DecodeArgs()
    a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim, a.rank, a.n_comp = 2, 32, 8, 64, 192, 4000
    a.n_splits, a.kernel = 10, 1
    assert lib.shard_decode_attn_workspace(ctypes.byref(a)) == 2 * 32 * 10 * (128 + 2) * 4
    assert lib.shard_decode_prepare_bytes(4, 192) < lib.shard_decode_prepare_bytes(8, 192)
    # an odd kv head count at head_dim 64 is refused before any launch
    assert lib.shard_decode_prepare(16, 16, 16, 16, 3, 64, 192, 16, 1 << 30, None) == -2
