"""ctypes binding of libshard_hip.so (the C ABI declared in include/shard_hip.h).

The library is built in-tree by ``shard_amd.build`` and loaded from this
package directory.  There is no fallback: if the library is missing or fails
to load, every kernel entry point raises ``ShardHipUnavailable``.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SHARD_HIP_LIB") or os.path.join(_HERE, "libshard_hip.so")

c_int32, c_int64, c_size_t, c_void_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
c_float = ctypes.c_float

ERRORS = {-1: "bad argument", -2: "unsupported shape", -3: "HIP error", -4: "workspace too small"}


class ShardHipUnavailable(RuntimeError):
    """libshard_hip.so could not be loaded (not built, or not loadable here)."""


class ShardHipError(RuntimeError):
    """A libshard_hip entry point returned a non-zero status."""

    def __init__(self, name, code, detail=""):
        self.code = code
        super().__init__(f"{name} failed with status {code} ({ERRORS.get(code, '?')}) {detail}".strip())


class DecodeArgs(ctypes.Structure):
    """Mirror of shard_decode_args (include/shard_hip.h)."""
    _fields_ = [
        ("batch", c_int32), ("n_q_heads", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32),
        ("rank", c_int32), ("n_comp", c_int32), ("compress_start", c_int32), ("pos_q", c_int32),
        ("q", c_void_p), ("inv_freq", c_void_p), ("k_coeffs", c_void_p), ("k_coeff_scale", c_void_p),
        ("k_basis", c_void_p), ("k_mean", c_void_p), ("prep", c_void_p), ("v_idx", c_void_p),
        ("v_codebook", c_void_p),
        ("v_ch", c_void_p),
        ("sink_k", c_void_p), ("sink_v", c_void_p), ("n_sink", c_int32),
        ("win_k", c_void_p), ("win_v", c_void_p), ("n_win", c_int32),
        ("dec_k", c_void_p), ("dec_v", c_void_p), ("n_dec", c_int32), ("dec_stride", c_int32),
        ("s_k", c_void_p), ("s_v", c_void_p), ("n_stream", c_int32), ("_pad0", c_int32),
        ("mask", c_void_p), ("mask_stride", c_int64),
        ("out", c_void_p), ("n_splits", c_int32), ("kernel", c_int32),
        ("pos_q_dev", c_void_p),
        ("n_stream_dev", c_void_p),
        ("v_group", c_int32), ("v_codebook_n", c_int32),
    ]


# (name, restype, argtypes) of every exported symbol
SIGNATURES = [
    ("shard_version", ctypes.c_char_p, []),
    ("shard_last_error", ctypes.c_char_p, []),
    ("shard_decode_args_size", c_size_t, []),
    ("shard_pca_project", c_int32, [c_void_p, c_int64, c_int32, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    ("shard_k_prepare", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("shard_pca_project_f32", c_int32, [c_void_p, c_int64, c_int32, c_int64, c_void_p, c_int32, c_void_p, c_int64, c_void_p]),
    ("shard_pca_project_rope", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_void_p]),
    ("shard_rope_phases", c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    ("shard_k_prepare_f32", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("shard_int4_quant_pack_workspace", c_size_t, [c_int64, c_int32]),
    ("shard_int4_quant_pack", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_fwht", c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    ("shard_vq_prepare_workspace", c_size_t, [c_int64, c_int32]),
    ("shard_vq_prepare", c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_vq_assign", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_int32, c_void_p, c_void_p]),
    ("shard_vq_table_bytes", c_size_t, [c_int32, c_int32]),
    ("shard_vq_scales", c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int64, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_size_t, c_void_p]),
    ("shard_vq_encode_table_workspace", c_size_t, [c_int64]),
    ("shard_vq_encode_table", c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int64, c_void_p, c_void_p, c_void_p,
                                        c_int32, c_void_p, c_size_t, c_int32, c_float, c_float, c_void_p,
                                        c_void_p, c_size_t, c_void_p]),
    ("shard_vq_table_build", c_int32, [c_void_p, c_int32, c_float, c_float, c_int32, c_void_p, c_size_t, c_void_p]),
    ("shard_vq_assign_table_workspace", c_size_t, [c_int64]),
    ("shard_vq_assign_table", c_int32, [c_void_p, c_int64, c_void_p, c_int32, c_void_p, c_size_t, c_int32, c_float,
                                        c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_kmeans_update_workspace", c_size_t, [c_int64, c_int32]),
    ("shard_kmeans_update_workspace_d", c_size_t, [c_int64, c_int32, c_int32]),
    ("shard_kmeans_update", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_stream_quant", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("shard_decode_prepare_bytes", c_size_t, [c_int32, c_int32]),
    ("shard_decode_prepare", c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_size_t, c_void_p]),
    ("shard_decode_supported", c_int32, [ctypes.POINTER(DecodeArgs)]),
    ("shard_decode_attn_workspace", c_size_t, [ctypes.POINTER(DecodeArgs)]),
    ("shard_decode_attn", c_int32, [ctypes.POINTER(DecodeArgs), c_void_p, c_size_t, c_void_p]),
    ("shard_decode_attn_noalloc", c_int32, [ctypes.POINTER(DecodeArgs), c_void_p]),
    # benchmark-only baseline (include/shard_bench.h)
    ("shard_bench_fp16_decode_workspace", c_size_t, [c_int32, c_int32, c_int32]),
    ("shard_bench_fp16_decode", c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_bench_fp16_decode_ld", c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int64, c_int32, c_void_p, c_void_p, c_size_t, c_void_p]),
    ("shard_kv_reconstruct", c_int32, [ctypes.POINTER(DecodeArgs), c_void_p, c_void_p, c_void_p]),
    ("shard_stream_dequant", c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("shard_stream_quant_qjl", c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("shard_stream_quant_kv", c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32] + [c_void_p] * 10 + [c_void_p]),
    ("shard_rope_stream_append", c_int32, [c_void_p] * 5 + [c_int64] + [c_int32] * 4 + [c_void_p] * 3 + [c_int32] + [c_void_p] * 10 + [c_void_p]),
    ("shard_rope_stream_append_dev", c_int32, [c_void_p] * 5 + [c_int64] + [c_int32] * 4 + [c_void_p] * 3 + [c_int32] + [c_void_p] * 10 + [c_void_p, c_int32] + [c_void_p]),
    ("shard_stream_dequant_qjl", c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
]

_lib = None
_load_error = None


def load():
    """Load (once) and return the ctypes handle of libshard_hip.so."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise ShardHipUnavailable(_load_error)
    if not os.path.exists(LIB_PATH):
        _load_error = f"{LIB_PATH} is missing: run shard_amd.build.build() (python -m shard_amd.build)"
        raise ShardHipUnavailable(_load_error)
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the host
        _load_error = f"cannot load {LIB_PATH}: {e}"
        raise ShardHipUnavailable(_load_error) from e
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.shard_decode_args_size() != ctypes.sizeof(DecodeArgs):
        raise ShardHipUnavailable("shard_decode_args layout mismatch between header and binding")
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except ShardHipUnavailable:
        return False


def check(name: str, code: int):
    if code != 0:
        detail = ""
        if code in (-3, -4) and _lib is not None:
            detail = _lib.shard_last_error().decode(errors="replace")
        raise ShardHipError(name, code, detail)
