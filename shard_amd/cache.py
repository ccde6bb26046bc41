"""shard.Cache on MI355X: a transformers Cache whose layers compress their KV.

API and state machine follow the reference's cache.py (Cache: 295-539,
CacheLayer: 64-292):
  prefill (q_len > 1)     fp16 K/V kept as-is (cache.py:142-147)
  first decode step       Cache.compress() of every layer (cache.py:149-151, 338-460):
                          K -> undo RoPE -> PCA (covariance eigh) -> DP bits -> int8
                          basis -> fp32 projection (MFMA) -> group quant -> int4 (HIP);
                          V -> Hadamard -> k-means VQ (HIP assign + update);
                          sink (4) and window (64) tokens stay fp16.
  decode tokens           8-bit Lloyd-Max stream (_streaming=True, HIP quantizer)
                          or fp16 decode_k/decode_v (cache.py:156-181)
  fused decode attention  attention.fused_attention_compressed (HIP kernel)
  unfused consumers       layer.keys / layer.values rebuild fp16 K/V on the GPU
                          (_ensure_dequant, cache.py:87-124; HIP reconstruct)
The compression's per-token work runs in HIP kernels of libshard_hip.so (undo
RoPE and centring, projection, int4 chain, Hadamard and VQ assignment, k-means
update); torch computes the column mean and the covariance GEMM of the fp32
rows, and the host a float64 eigendecomposition of the (p, p) covariance.
CPU tensors are rejected.
"""
import torch
from transformers.cache_utils import Cache as HFCache, CacheLayerMixin

from . import host, ops


def _nb(t):
    return t.nelement() * t.element_size()


# Stream buffers (cap, ...) of a layer: 8-bit codes and the fp16 rows the
# reference's dequantization yields (cache.py:275-278; written once per token,
# read by the decode kernel), fp16 norms; with _stream_qjl the residual signs
# and scales (cache.py:234-240).
_STREAM_BUFS = ("k_idx_buf", "v_idx_buf", "k_norm_buf", "v_norm_buf", "k_deq_buf", "v_deq_buf")
_STREAM_BUFS_QJL = _STREAM_BUFS + ("k_qsign_buf", "v_qsign_buf", "k_qscale_buf", "v_qscale_buf")


def _stream_buf_shape(name, B, G, D):
    """(per-token shape, dtype) of stream buffer ``name``."""
    if name.endswith("_idx_buf") or name.endswith("_qsign_buf"):
        return (B, G, D), torch.uint8
    if name.endswith("_deq_buf"):
        return (B, G, D), torch.float16
    return (B, G), torch.float16  # norms, QJL scales


class CacheLayer(CacheLayerMixin):
    """One layer's cache (cache.py:64-292)."""

    is_sliding = False
    is_compileable = False

    def __init__(self, layer_idx):
        self.layer_idx = layer_idx
        self._keys = None
        self._values = None
        self._prefilled = False
        self._seq_len = 0
        self._cache_ref = None
        self._needs_decompress = False
        self._gpu_compressed = None
        self.is_initialized = False

    # -- lazy per-layer materialization (cache.py:74-136) -------------------
    def _lazy_evict(self):
        c = self._cache_ref
        if c is None or not c._lazy_per_layer:
            return
        last = c._last_accessed_layer
        if last != -1 and last != self.layer_idx:
            prev = c.layers[last]
            if getattr(prev, "_gpu_compressed", None) is not None:
                prev._keys = None
                prev._values = None
                prev._needs_decompress = True
        c._last_accessed_layer = self.layer_idx

    def _ensure_dequant(self):
        if not self._needs_decompress:
            return
        gc = self._gpu_compressed
        if gc is None:
            return
        B = gc["batch"]
        k_mid, v_mid = ops.kv_reconstruct(gc, B)
        parts_k = [gc["sink_k"], k_mid, gc["win_k"]]
        parts_v = [gc["sink_v"], v_mid, gc["win_v"]]
        sk, sv = self._dequant_stream(gc, B)
        if sk is not None:
            parts_k.append(sk)
            parts_v.append(sv)
        if "decode_k" in gc:
            parts_k.append(gc["decode_k"])
            parts_v.append(gc["decode_v"])
        self._keys = torch.cat(parts_k, dim=2)
        self._values = torch.cat(parts_v, dim=2)
        self._needs_decompress = False

    @property
    def keys(self):
        self._lazy_evict()
        self._ensure_dequant()
        return self._keys

    @keys.setter
    def keys(self, v):
        self._keys = v

    @property
    def values(self):
        self._lazy_evict()
        self._ensure_dequant()
        return self._values

    @values.setter
    def values(self, v):
        self._values = v

    # -- update (cache.py:138-191) -----------------------------------------
    def update(self, key_states, value_states, *args, **kwargs):
        seq_new = key_states.shape[2]
        c = self._cache_ref
        self.is_initialized = True
        if seq_new > 1 and not self._prefilled:
            self._prefilled = True
            self._seq_len = seq_new
            self._keys = key_states
            self._values = value_states
            return key_states, value_states

        if self.layer_idx == 0 and c is not None and not c._compressed:
            c.compress()

        self._lazy_evict()
        gc = self._gpu_compressed

        if gc is not None and c._streaming:
            for t in range(seq_new):
                self._stream_append(key_states[:, :, t:t + 1, :], value_states[:, :, t:t + 1, :])
            self._seq_len += seq_new
            self._needs_decompress = True
            if getattr(c, "_fused_decode_update", False):
                return key_states, value_states
            self._ensure_dequant()
            return self._keys, self._values

        if gc is not None:
            if "decode_k" in gc:
                gc["decode_k"] = torch.cat([gc["decode_k"], key_states], dim=2)
                gc["decode_v"] = torch.cat([gc["decode_v"], value_states], dim=2)
            else:
                gc["decode_k"] = key_states.contiguous()
                gc["decode_v"] = value_states.contiguous()
            self._seq_len += seq_new
            self._needs_decompress = True
            if getattr(c, "_fused_decode_update", False):
                return key_states, value_states
            self._ensure_dequant()
            return self._keys, self._values

        self._ensure_dequant()
        self._seq_len += seq_new
        if self._keys is not None:
            self._keys = torch.cat([self._keys, key_states], dim=2)
            self._values = torch.cat([self._values, value_states], dim=2)
        else:
            self._keys = key_states
            self._values = value_states
        return self._keys, self._values

    # -- decode stream (cache.py:193-279) ----------------------------------
    def _stream_rows(self, B, G, D, dev, min_cap=0, row=None):
        """Device addresses of the next stream row of every buffer, growing the
        buffers by doubling when full (cache.py:220-230), and to at least
        min_cap rows.  row: the row whose addresses are returned instead of the
        next one (0: the buffers' bases).  Returns (codebook tensors, k row
        pointers, v row pointers, QJL pointers)."""
        gc = self._gpu_compressed
        c = self._cache_ref
        bits, qjl = int(c._stream_bits), bool(c._stream_qjl)
        if not 1 <= bits <= 8:
            raise ValueError(f"_stream_bits must be in 1..8 (uint8 codes), got {bits}")
        if "signs" not in gc:
            gc["signs"] = host.stream_signs(self.layer_idx, D).to(dev)
        if gc.get("stream_bits") != bits:
            gc["stream_codebook"] = host.lloyd_max_codebook(D, bits).to(dev)
            gc["stream_bits"] = bits
        s = gc.get("stream_n", 0) // B
        names = _STREAM_BUFS_QJL if qjl else _STREAM_BUFS
        if (gc.get("_stream_cap", 0) <= max(s, min_cap - 1)
                or (qjl and "k_qsign_buf" not in gc)):
            cap = max(s + 1, min_cap, 16 if gc.get("_stream_cap", 0) == 0 else 2 * gc["_stream_cap"])
            for name in names:
                per_token, dtype = _stream_buf_shape(name, B, G, D)
                buf = gc.get(name)
                new = torch.empty((cap, *per_token), device=dev, dtype=dtype)
                if buf is not None:
                    new[:buf.shape[0]].copy_(buf)
                gc[name] = new
            gc["_stream_cap"] = cap
        # row s of each buffer, by address: codes and fp16 rows hold B G D
        # entries per token, norms and QJL scales B G (fp16).  The buffers'
        # base addresses are kept until the buffers change.
        base = gc.get("_stream_base")
        if base is None or base[0] is not gc["k_idx_buf"] or base[1] != qjl:
            ptr = lambda name: gc[name].data_ptr() if name in gc else None
            base = (gc["k_idx_buf"], qjl, tuple(ptr(n) for n in (
                "k_idx_buf", "k_norm_buf", "k_deq_buf", "v_idx_buf", "v_norm_buf", "v_deq_buf",
                "k_qsign_buf", "k_qscale_buf", "v_qsign_buf", "v_qscale_buf")))
            gc["_stream_base"] = base
        ki, kn, kd, vi, vn, vd, kqs, kqc, vqs, vqc = base[2]
        rows = B * G
        if row is not None:
            s = row
        p8, p16, n16 = s * rows * D, 2 * s * rows * D, 2 * s * rows
        kp = (ki + p8, kn + n16, kd + p16)
        vp = (vi + p8, vn + n16, vd + p16)
        qp = (kqs + p8, kqc + n16, vqs + p8, vqc + n16) if qjl else (None, None, None, None)
        return (gc["signs"], gc["stream_codebook"]), kp, vp, qp

    def _stream_append(self, k, v):
        """Quantize one decode token (B, G, 1, D) of K and V into the 8-bit
        stream buffers (growable, doubling, as cache.py:220-230)."""
        gc = self._gpu_compressed
        if getattr(self._cache_ref, "_graph", None) is not None:
            # this launch takes the row by address, which a replay would repeat
            raise RuntimeError("under a decode graph tokens are appended by fused_rope_append "
                               "(fp16 q, k, v, cos and sin)")
        B, G, _, D = k.shape
        cbs, kp, vp, qp = self._stream_rows(B, G, D, k.device)
        kx = k.reshape(B, G, D)
        vx = v.reshape(B, G, D)
        if not kx.is_contiguous():
            kx = kx.contiguous()
        if not vx.is_contiguous():
            vx = vx.contiguous()
        ops.stream_quant_kv_at(kx, vx, *cbs, *kp, *vp, *qp)
        gc["stream_n"] = gc.get("stream_n", 0) + B

    def fused_rope_append(self, q, k, v, cos, sin):
        """One decode token of a streaming compressed layer: RoPE of q and k
        (transformers' fp16 apply_rotary_pos_emb) and the rotated k and v
        appended to the stream, in one launch - the patched forward's
        apply_rotary_pos_emb + update (attention.py:376-381).  q (B, H, 1, D),
        k and v (B, G, 1, D), cos and sin (B or 1, 1, D), all fp16 and contiguous
        in memory; cos and sin may have batch 1 (positions shared by the
        batch).  Returns q after RoPE as (B, H, D)."""
        gc = self._gpu_compressed
        B, H, _, D = q.shape
        G = k.shape[1]
        self._lazy_evict()
        graph = getattr(self._cache_ref, "_graph", None)
        # under a decode graph the token's row comes from the graph's device
        # counter, so the launch takes the buffers' bases
        cbs, kp, vp, qp = self._stream_rows(B, G, D, q.device, row=0 if graph else None)
        # q after RoPE goes to a per-layer buffer: this step's attention reads it
        # (stream-ordered before the next step's append rewrites it)
        q_out = gc.get("_q_rope")
        if q_out is None or q_out.shape != (B, H, D) or q_out.device != q.device:
            q_out = torch.empty(B, H, D, dtype=torch.float16, device=q.device)
            gc["_q_rope"] = q_out
        c16 = lambda t, *shape: t.reshape(*shape).contiguous()
        Bc = cos.shape[0]  # 1 when the batch shares its positions
        dev_row = {} if graph is None else {"row_dev": graph.rows[0:1], "row_cap": gc["_stream_cap"]}
        ops.rope_stream_append_at(c16(q, B, H, D), c16(k, B, G, D), c16(v, B, G, D),
                                  c16(cos, Bc, D), c16(sin, Bc, D), *cbs, q_out, *kp, *vp, *qp,
                                  **dev_row)
        gc["stream_n"] = gc.get("stream_n", 0) + B
        self._seq_len += 1
        self._needs_decompress = True
        return q_out

    def _dequant_stream(self, gc, B, nkv=None, hd=None):
        n = gc.get("stream_n", 0)
        if n == 0 or "k_idx_buf" not in gc:
            return None, None
        s = n // B
        sk = gc["k_deq_buf"][:s]
        sv = gc["v_deq_buf"][:s]
        return sk.permute(1, 2, 0, 3).contiguous(), sv.permute(1, 2, 0, 3).contiguous()

    # -- HF Cache API glue (cache.py:281-292; TF 5.x additions) ----------------
    def get_seq_length(self):
        return self._seq_len

    def get_max_length(self):
        return -1

    def get_max_cache_shape(self):
        return None

    def get_mask_sizes(self, query_length, *args, **kwargs):
        return self._seq_len + query_length, 0

    def lazy_initialization(self, *args, **kwargs):
        pass

    def reorder_cache(self, beam_idx):
        """Beam reordering (cache.py:287-292).  The reference rebuilds the
        dequantized K/V and selects their batch rows, and leaves the compressed
        representation as it was, so its next decode step (which reads it) sees
        the old row order.  Here the compressed layer's per-row tensors are
        selected, so every later step runs on the reordered beams; dequantized
        K/V that are current are selected too, and stale ones are dropped and
        rebuilt from the selected rows at their next access.  Each batch row is
        rebuilt from its own rows only, so that equals the reference's
        rebuild-then-select, without a full rebuild at every beam step."""
        if getattr(self._cache_ref, "_graph", None) is not None:
            # a captured decode step holds the addresses of the rows reordered here
            raise RuntimeError("reorder_cache while a decode graph is open: close() it first")
        if self._needs_decompress and self._gpu_compressed is not None:
            self._keys = self._values = None
        if self._keys is not None:
            self._keys = self._keys.index_select(0, beam_idx.to(self._keys.device))
        if self._values is not None:
            self._values = self._values.index_select(0, beam_idx.to(self._values.device))
        if self._gpu_compressed is not None:
            reorder_rows(self._gpu_compressed, beam_idx)


class Cache(HFCache):
    """KV cache compression (cache.py:295-539).
    Prefill: per-layer PCA on K (RoPE removed, int4 coefficients + int8 basis)
    + Hadamard + k-means VQ on V; sink (4) + window (64) kept fp16.
    Decode: optional 8-bit Lloyd-Max per-token stream (``_streaming``)."""

    def __init__(self, head_dim=128, num_layers=32, n_kv_heads=8, device="cuda",
                 k_target_cr=20.0, max_rank_k=192,
                 v_vq_group_size=4, v_vq_codebook_size=256,
                 sink_tokens=4, residual_window=64, rope_inv_freq=None):
        # V subvectors of 1, 2, 4 or 8 values (the assignment and update kernels'
        # widths) and at most 256 centroids (one byte per index, as the
        # reference's v_indices_u8, cache.py:442): refused here rather than
        # after a layer's compression
        if v_vq_group_size not in (1, 2, 4, 8) or head_dim % v_vq_group_size:
            raise ValueError(f"v_vq_group_size={v_vq_group_size}: this build takes 1, 2, 4 or 8 "
                             f"dividing head_dim={head_dim}")
        if not 1 <= v_vq_codebook_size <= 256:
            raise ValueError(f"v_vq_codebook_size={v_vq_codebook_size}: indices are one byte "
                             "(1..256 centroids)")
        self.head_dim = head_dim
        self._num_layers = num_layers
        self._n_kv_heads = n_kv_heads
        self._per_layer_dim = n_kv_heads * head_dim
        self._k_target_cr = k_target_cr
        self._max_rank_k = max_rank_k
        self._v_vq_group_size = v_vq_group_size
        self._v_vq_codebook_size = v_vq_codebook_size
        self._sink_tokens = sink_tokens
        self._residual_window = residual_window
        self._rope_inv_freq = rope_inv_freq
        self._device = device
        self._streaming = False
        self._stream_bits = 8
        self._stream_qjl = False
        self._lazy_per_layer = True
        self._full_fused = False
        self._last_accessed_layer = -1
        self._compressed = False
        self._compressed_layers = {}
        self._fused_decode_update = False
        # decode-attention knobs of the HIP kernel (0 = automatic split count)
        self._n_splits = 0
        self._decode_kernel = 0  # decode split kernel: 0 automatic, 1 row-split, 2 token-tiled
        self._graph = None  # the DecodeGraph whose device counters decode steps use
        self._basis_override = None  # {layer_idx: (1024, rank) fp32} to pin the PCA basis
        super().__init__(layers=[CacheLayer(i) for i in range(num_layers)])
        for l in self.layers:
            l._cache_ref = self

    @classmethod
    def from_model(cls, model, k_target_cr=16.0, **kwargs):
        cfg = model.config
        hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        return cls(head_dim=hd, num_layers=cfg.num_hidden_layers,
                   n_kv_heads=getattr(cfg, "num_key_value_heads", cfg.num_attention_heads),
                   device=str(next(model.parameters()).device),
                   k_target_cr=k_target_cr,
                   rope_inv_freq=host.get_rope_inv_freq(model), **kwargs)

    # -- compression (cache.py:338-460) -----------------------------------
    def compress(self):
        if self._compressed:
            return
        k0 = self.layers[0]._keys
        if k0 is None:
            return
        B, _, seq, _ = k0.shape
        sink, win = self._sink_tokens, self._residual_window
        if seq <= sink + win + 4:
            return
        if k0.dtype != torch.float16:
            # the compressed format keeps fp16 segments and fp16 operands, as
            # the reference's does (cache.py:96-113, 430-449; its example and
            # README load the model in float16)
            raise TypeError(f"shard_amd.Cache compresses fp16 K/V (a float16 model); got {k0.dtype}")
        if not k0.is_cuda:
            raise ops.ShardHipUnavailable("shard_amd.Cache compresses on the GPU only")
        for li in range(self._num_layers):
            layer = self.layers[li]
            if layer._keys is None:
                continue
            layer._gpu_compressed = compress_layer(self, layer._keys, layer._values, li)
            layer._keys = None
            layer._values = None
            layer._needs_decompress = True
        self._compressed = True

    # -- memory accounting (cache.py:462-539) ------------------------------
    def memory_bytes(self):
        """Compressed bytes as the reference counts them (cache.py:462-497): its
        key set, under this format's names (``v_indices`` holds what the
        reference calls ``v_indices_u8``), stream codes at their bit width.
        ``device_bytes`` counts every tensor this format keeps resident."""
        total = 0
        has_gc = False
        for l in self.layers:
            gc = l._gpu_compressed
            if gc is None:
                continue
            has_gc = True
            total += sum(_nb(gc[k]) for k in
                         ("k_coeffs", "k_coeff_scale", "k_basis_q", "k_basis_scale", "k_mean",
                          "v_packed", "sink_k", "sink_v", "win_k", "win_v"))
            for k in ("k_basis_f16", "k_mean_f16", "v_indices", "v_centroids_f16", "v_ch_f16"):
                if k in gc:
                    total += _nb(gc[k])
            for k, v in gc.items():
                if k.endswith("_f32") and torch.is_tensor(v):
                    total += _nb(v)
            total += _nb(gc["v_qdata"]["ch_maxabs"])
            if gc["v_qdata"].get("centroids") is not None:
                total += _nb(gc["v_qdata"]["centroids"])
            if "k_idx_buf" in gc:
                s = gc.get("stream_n", 0) // max(gc.get("batch", 1), 1)
                bpv = self._stream_bits / 8.0
                for k in ("k_idx_buf", "v_idx_buf"):
                    total += int(gc[k][:s].nelement() * bpv)
                for k in ("k_norm_buf", "v_norm_buf"):
                    total += _nb(gc[k][:s])
            if "decode_k" in gc:
                total += _nb(gc["decode_k"]) + _nb(gc["decode_v"])
        if has_gc:
            return total
        return sum(_nb(l._keys) + _nb(l._values) for l in self.layers if l._keys is not None)

    def device_bytes(self):
        """Every device tensor the compressed layers keep (each counted once),
        including the decode kernel's per-layer operands and the dequantized
        stream rows; stream codes at their bit width, QJL signs at 1 bit."""
        total = 0
        has_gc = False
        for l in self.layers:
            gc = l._gpu_compressed
            if gc is None:
                continue
            has_gc = True
            seen = set()
            for k, v in gc.items():
                if (torch.is_tensor(v) and v.data_ptr() not in seen and not k.endswith("_buf")
                        and not k.startswith("_")):  # "_" keys: per-step scratch
                    seen.add(v.data_ptr())
                    total += _nb(v)
            if "k_idx_buf" in gc:
                s = gc.get("stream_n", 0) // max(gc.get("batch", 1), 1)
                bpv = self._stream_bits / 8.0
                for k in ("k_idx_buf", "v_idx_buf"):
                    total += int(gc[k][:s].nelement() * bpv)
                for k in ("k_norm_buf", "v_norm_buf", "k_deq_buf", "v_deq_buf"):
                    total += _nb(gc[k][:s])
                if "k_qsign_buf" in gc:  # QJL: 1 bit per element + fp16 scale per token
                    for k in ("k_qsign_buf", "v_qsign_buf"):
                        total += gc[k][:s].nelement() // 8
                    for k in ("k_qscale_buf", "v_qscale_buf"):
                        total += _nb(gc[k][:s])
        if has_gc:
            return total
        return sum(_nb(l._keys) + _nb(l._values) for l in self.layers if l._keys is not None)

    def clean_memory_bytes(self):
        """Storage-only compressed KV size (same fields as cache.py:499-516)."""
        total = 0
        has_gc = False
        for l in self.layers:
            gc = l._gpu_compressed
            if gc is None:
                continue
            has_gc = True
            total += sum(_nb(gc[k]) for k in
                         ("k_coeffs", "k_coeff_scale", "k_basis_q", "k_basis_scale", "k_mean",
                          "v_packed", "sink_k", "sink_v", "win_k", "win_v"))
            total += _nb(gc["v_qdata"]["ch_maxabs"])
            if gc["v_qdata"].get("centroids") is not None:
                total += _nb(gc["v_qdata"]["centroids"])
        if has_gc:
            return total
        return sum(_nb(l._keys) + _nb(l._values) for l in self.layers if l._keys is not None)

    def _fp16_seq(self, with_stream):
        gc = self.layers[0]._gpu_compressed
        if gc is not None:
            return (gc["n_compress"] + self._sink_tokens + self._residual_window
                    + (gc.get("stream_n", 0) if with_stream else 0))
        if self._compressed_layers:
            return (next(iter(self._compressed_layers.values()))["n_compress"]
                    + self._sink_tokens + self._residual_window)
        if self.layers[0]._keys is not None:
            return self.layers[0]._keys.shape[2]
        return 0

    def fp16_equivalent_bytes(self):
        """fp16 K+V bytes of the same context, as the reference counts them
        (cache.py:518-528): one batch row, plus ``stream_n`` (stream tokens x
        batch rows) stream positions.  ``fp16_equivalent_bytes_all_rows`` counts
        every batch row."""
        return self._fp16_seq(True) * self._n_kv_heads * self.head_dim * 4 * self._num_layers

    def fp16_equivalent_bytes_all_rows(self):
        """fp16 K+V bytes of the whole batch (every row, stream tokens once per row)."""
        gc = self.layers[0]._gpu_compressed
        if gc is not None:
            batch = gc.get("batch", 1)
            seq = (gc["n_compress"] + self._sink_tokens + self._residual_window
                   + gc.get("stream_n", 0) // max(batch, 1))
        elif self.layers[0]._keys is not None:
            batch, seq = self.layers[0]._keys.shape[0], self.layers[0]._keys.shape[2]
        else:
            return 0
        return batch * seq * self._n_kv_heads * self.head_dim * 4 * self._num_layers

    def compress_ratio(self):
        return self.fp16_equivalent_bytes() / max(self.memory_bytes(), 1)

    def clean_compress_ratio(self):
        """cache.py:534-539: one batch row of fp16 over the stored bytes."""
        if self.layers[0]._gpu_compressed is not None:
            fp16_bytes = (self._fp16_seq(False) * self._n_kv_heads * self.head_dim * 4
                          * self._num_layers)
            return fp16_bytes / max(self.clean_memory_bytes(), 1)
        return self.compress_ratio()

    def clean_compress_ratio_all_rows(self):
        """fp16 bytes of every batch row over the stored bytes (the storage
        compression of a batch > 1)."""
        gc = self.layers[0]._gpu_compressed
        if gc is not None:
            return gc.get("batch", 1) * self.clean_compress_ratio()
        return self.fp16_equivalent_bytes_all_rows() / max(self.memory_bytes(), 1)


def _undo_rope_mean(k_full: torch.Tensor, start: int, end: int, inv_freq,
                    chunk: int = 2048) -> torch.Tensor:
    """Column mean (over batch rows and tokens [start, end)) of the keys with
    RoPE undone, in fp32 as cache.py:370-374 computes it, a token chunk at a
    time; (G * D,) with column g * D + d."""
    B, G, _, D = k_full.shape
    acc = torch.zeros(G, D, dtype=torch.float32, device=k_full.device)
    for t0 in range(start, end, chunk):
        t1 = min(end, t0 + chunk)
        km = k_full[:, :, t0:t1, :].float()
        if inv_freq is not None:
            km = host.undo_rope(km, torch.arange(t0, t1, device=k_full.device),
                                inv_freq.to(k_full.device))
        acc += km.sum(dim=(0, 2))
    return acc.reshape(-1) / (B * (end - start))


def _covariance(x16: torch.Tensor, chunk: int = 1 << 15) -> torch.Tensor:
    """X^T X / n of the rows (fp16 or fp32) in fp32, a row chunk at a time."""
    n, p = x16.shape
    cov = torch.zeros(p, p, dtype=torch.float32, device=x16.device)
    for i in range(0, n, chunk):
        xc = x16[i:i + chunk].float()
        cov.addmm_(xc.t(), xc)
    return cov / n


def _column_energy(x16: torch.Tensor, basis: torch.Tensor, chunk: int = 1 << 15) -> torch.Tensor:
    """mean over rows of (x @ basis)^2 (the variances along a supplied basis)."""
    acc = torch.zeros(basis.shape[1], dtype=torch.float32, device=x16.device)
    for i in range(0, x16.shape[0], chunk):
        acc += (x16[i:i + chunk].float() @ basis).pow(2).sum(dim=0)
    return acc / x16.shape[0]


def _eigh_top(cov_host: torch.Tensor, rank: int):
    """Top-`rank` eigenvectors and eigenvalues of a host float64 (p, p)
    covariance (symmetric eigendecomposition, deterministic)."""
    evals, evecs = torch.linalg.eigh(cov_host)
    return evecs.flip(1)[:, :rank].float(), evals.flip(0)[:rank].clamp(min=0.0).float()


def pca_basis_cov(cov: torch.Tensor, rank: int):
    """Top-`rank` eigenvectors of a (p, p) covariance and their eigenvalues, by
    a float64 symmetric eigendecomposition on the host (deterministic)."""
    evecs, evals = _eigh_top(cov.double().cpu(), rank)
    return evecs.to(cov.device), evals.to(cov.device)


_host_pool = None


def _host_worker():
    """One background thread for host work that overlaps the GPU (the PCA
    eigendecomposition runs there while the V codec's kernels run)."""
    global _host_pool
    if _host_pool is None:
        import concurrent.futures
        _host_pool = concurrent.futures.ThreadPoolExecutor(max_workers=1, thread_name_prefix="shard-host")
    return _host_pool


def pca_basis(centered: torch.Tensor, rank: int):
    """Top-`rank` principal directions of the centered rows and their variances
    (S^2 / n), the quantities _compress_k takes from svd_lowrank(q=rank,
    niter=24) (cache.py:376-378).  The reference's randomized subspace iteration
    converges to this subspace; here it is computed exactly and
    deterministically: the fp32 covariance X^T X / n on the GPU (one GEMM), then
    a float64 symmetric eigendecomposition of the (p, p) matrix on the host."""
    n = centered.shape[0]
    return pca_basis_cov((centered.t() @ centered) / n, rank)


def compress_layer(cache: Cache, k_full: torch.Tensor, v_full: torch.Tensor, li: int,
                   basis=None, debug=None) -> dict:
    """Compress one layer's prefill K/V (B, G, T, D) fp16 into the device format.

    _compress_k (cache.py:368-396), _compress_v (398-404), _build_gpu_format
    (406-454).  The projection runs on the fp32 MFMA GEMM, the integer chain, the
    Hadamard/normalization, the k-means assignment and update in HIP kernels.
    ``debug``: a dict that receives the fp32 projection ``proj`` (rows, keep)
    and the bit allocation ``alloc`` (for parity tests).
    """
    B, G, seq, D = k_full.shape
    dev = k_full.device
    sink, win = cache._sink_tokens, cache._residual_window
    start, end = sink, seq - win
    n_comp = end - start
    inv_freq = cache._rope_inv_freq
    torch.manual_seed(42 + li)

    # ---- K: undo RoPE and centring (shard_k_prepare_f32: the fp32 rows of
    # (flat - mean), cache.py:370-392), PCA basis, DP bits, int8 basis
    p_dim = G * D
    n = B * n_comp
    invf = (inv_freq.to(dev, torch.float32) if inv_freq is not None
            else torch.zeros(D // 2, dtype=torch.float32, device=dev))  # phase 0: no rotation
    k_full = k_full.contiguous()
    mean = _undo_rope_mean(k_full, start, end, inv_freq)
    centered = ops.k_prepare(k_full, start, n_comp, invf, mean, out_dtype=torch.float32)  # (n, p_dim)
    rank = min(cache._max_rank_k, p_dim, n - 1)
    if basis is None and cache._basis_override is not None:
        basis = cache._basis_override.get(li)
    eig_job = None
    if basis is None:
        # the host eigendecomposition overlaps the V codec's GPU work below
        cov_host = _covariance(centered).double().cpu()
        eig_job = _host_worker().submit(_eigh_top, cov_host, rank)
    else:
        basis = basis.to(dev, torch.float32)[:, :rank]
        eig = _column_energy(centered, basis)

    # ---- V: Hadamard -> channel max -> 4-dim subvectors -> k-means (256)
    x, ch32, ch16 = ops.vq_prepare(v_full[:, :, start:end, :].reshape(B * G, n_comp, D),
                                   cache._v_vq_group_size)
    centroids, idx = ops.kmeans(x, cache._v_vq_codebook_size, n_iter=30, seed=42)
    del x
    if eig_job is not None:
        basis, eig = (t.to(dev) for t in eig_job.result())
    budget = max(64, int(p_dim * 16 / cache._k_target_cr))
    alloc = host.dp_bit_allocation(eig, budget)
    keep = sum(1 for b in alloc if b > 0)
    if keep & 1:
        keep -= 1
    if keep == 0:
        # every component dropped (a budget below one group's cheapest option):
        # the reference keeps them all, with zero coefficients, so the keys
        # decode to the mean (_build_gpu_format takes keep = len(k_alloc),
        # cache.py:412); an even count, as every stored rank here
        keep = len(alloc) - (len(alloc) & 1)
    basis = basis[:, :keep].contiguous()
    alloc = alloc[:keep]
    col_max = basis.abs().max(dim=0).values.clamp(min=1e-6)
    scale = col_max / 127.0
    basis_q = (basis / scale).round().clamp(-127, 127).to(torch.int8)
    basis_deq = basis_q.float() * scale.float()                  # (p_dim, keep)

    # ---- projection on fp32 MFMA, fp32 operands as the reference's
    # (flat - mean) @ (basis_q * scale) (cache.py:392); columns padded to 32
    keep32 = ((keep + 31) // 32) * 32
    bt = torch.zeros(keep32, p_dim, dtype=torch.float32, device=dev)
    bt[:keep] = basis_deq.t()
    proj = ops.pca_project_f32(centered, bt)[:, :keep].contiguous()
    del centered
    bits = torch.tensor(alloc, dtype=torch.int32, device=dev)
    chain = ops.int4_quant_pack(proj, bits)
    if debug is not None:
        debug["proj"], debug["alloc"] = proj, list(alloc)
    del proj

    ng = D // cache._v_vq_group_size
    v_idx = idx.to(torch.uint8)
    v_indices = v_idx.view(B, G, n_comp, ng)

    k_scale_h = scale.half()
    k_basis_f16 = (basis_q.to(torch.float16) * k_scale_h.to(torch.float16)).contiguous()
    cs16 = chain["coeff_scale"].half()
    gc = {
        "k_coeffs": chain["packed"],
        "k_coeff_scale": cs16,
        "k_coeffs_shape": (B * n_comp, keep),
        "k_basis_q": basis_q,
        "k_basis_scale": k_scale_h,
        "k_basis_f16": k_basis_f16,
        "k_mean": mean.half(),
        "k_mean_f16": mean.half().contiguous(),
        "k_alloc": alloc,
        "v_qdata": {"centroids": centroids.half(), "packed": v_idx, "ch_maxabs": ch16,
                    "shape": (B * G, n_comp, D), "group_size": cache._v_vq_group_size,
                    "bits": 8, "n_orig": v_idx.numel()},
        "v_packed": v_idx,
        "v_indices": v_indices,
        "v_centroids_f16": centroids.half().contiguous(),
        "v_ch_f16": ch16.view(B, G, D),
        "sink_k": k_full[:, :, :sink, :].contiguous(),
        "sink_v": v_full[:, :, :sink, :].contiguous(),
        "win_k": k_full[:, :, end:, :].contiguous(),
        "win_v": v_full[:, :, end:, :].contiguous(),
        "n_compress": n_comp, "batch": B, "compress_start": start,
        "n_kv": G, "head_dim": D, "rank": keep,
    }
    if B == 1:
        gc["v_indices_u8"] = v_indices.view(G, n_comp, ng)
    finalize_format(gc, inv_freq, dev)
    return gc


def reorder_rows(gc: dict, beam_idx) -> None:
    """Select the batch rows `beam_idx` of every per-row tensor of a compressed
    layer (coefficients, V indices and channel scales, fp16 segments, stream
    rows); the basis, mean, codebooks and decode operands are shared by the
    rows and stay."""
    B = gc["batch"]
    idx = beam_idx.to(gc["k_coeffs"].device, torch.long)
    if idx.numel() != B:
        raise ValueError(f"reorder_cache: {idx.numel()} indices for batch {B}")
    n = gc["n_compress"]
    rows = lambda t, dim=0: t.index_select(dim, idx).contiguous()
    same_pad = gc.get("k_coeffs_pad") is gc["k_coeffs"]
    gc["k_coeffs"] = rows(gc["k_coeffs"].view(B, -1)).view(-1)
    if same_pad:
        gc["k_coeffs_pad"] = gc["k_coeffs"]
    elif "k_coeffs_pad" in gc:
        gc["k_coeffs_pad"] = rows(gc["k_coeffs_pad"].view(B, -1)).view(-1)
    gc["v_indices"] = rows(gc["v_indices"])
    gc["v_packed"] = gc["v_indices"].view(-1)
    gc["v_ch_f16"] = rows(gc["v_ch_f16"])
    qd = gc["v_qdata"]
    qd["packed"] = gc["v_packed"]
    qd["ch_maxabs"] = gc["v_ch_f16"].view(B * gc["n_kv"], -1)
    for k in ("sink_k", "sink_v", "win_k", "win_v", "decode_k", "decode_v"):
        if k in gc:
            gc[k] = rows(gc[k])
    for k in _STREAM_BUFS_QJL:
        if k in gc:
            gc[k] = rows(gc[k], 1)
    assert gc["v_indices"].shape[2] == n
    for k in ("_decode_call", "_stream_base", "_q_rope"):  # held the old tensors or addresses
        gc.pop(k, None)


def finalize_format(gc: dict, inv_freq, dev):
    """Derived device tensors of the decode kernel: rank padded to a multiple of
    32 (zero nibbles / zero basis columns), inverse frequencies on the device."""
    n_total, keep = gc["k_coeffs_shape"]
    rank_pad = ((keep + 31) // 32) * 32
    gc["rank_pad"] = rank_pad
    if rank_pad == keep:
        gc["k_coeffs_pad"] = gc["k_coeffs"]
        gc["k_basis_pad"] = gc["k_basis_f16"]
        gc["k_coeff_scale_pad"] = gc["k_coeff_scale"]
    else:
        packed = gc["k_coeffs"][: n_total * keep // 2].view(n_total, keep // 2)
        pad = torch.full((n_total, rank_pad // 2), 0x88, dtype=torch.uint8, device=dev)
        pad[:, : keep // 2] = packed
        gc["k_coeffs_pad"] = pad.reshape(-1)
        bp = torch.zeros(gc["k_basis_f16"].shape[0], rank_pad, dtype=torch.float16, device=dev)
        bp[:, :keep] = gc["k_basis_f16"]
        gc["k_basis_pad"] = bp
        cp = torch.zeros(rank_pad, dtype=torch.float16, device=dev)
        cp[:keep] = gc["k_coeff_scale"]
        gc["k_coeff_scale_pad"] = cp
    if inv_freq is None:
        inv_freq = torch.zeros(gc["head_dim"] // 2)
    gc["inv_freq_dev"] = inv_freq.to(dev, torch.float32).contiguous()
    # decode-kernel operands for the shapes the fused kernel takes (head_dim
    # 128, or 64 with an even kv head count, rank up to 256, a finite rebuild
    # constant); other layers decode through kv_reconstruct and the model's
    # own attention
    hd, G = gc["head_dim"], gc["n_kv"]
    gc["decode_prep"] = None
    gc.pop("decode_refusal", None)
    # the fused value stage reads 4-value subvectors from a 256-row codebook:
    # a smaller codebook is padded with rows no index names
    cb = gc["v_centroids_f16"]
    gc.pop("v_centroids_pad", None)
    if cb.shape[1] == 4:
        if cb.shape[0] == 256:
            gc["v_centroids_pad"] = cb
        else:
            pad = torch.zeros(256, 4, dtype=torch.float16, device=cb.device)
            pad[: cb.shape[0]] = cb
            gc["v_centroids_pad"] = pad
    if "v_centroids_pad" not in gc:
        gc["decode_refusal"] = f"V subvectors of {cb.shape[1]} values (the fused kernel takes 4)"
    elif (hd == 128 or (hd == 64 and G % 2 == 0)) and rank_pad <= 256:
        cmax = ops.decode_constant_max(gc["k_basis_pad"], gc["k_coeff_scale_pad"], gc["k_mean_f16"])
        if cmax <= ops.DECODE_CONSTANT_LIMIT:  # False for NaN
            gc["decode_prep"] = ops.decode_prepare(gc)
        else:
            gc["decode_refusal"] = f"rebuild constant {cmax:.4g} not finite or beyond fp32"
