"""Torch-facing wrappers of the HIP hot path, with the reference's native op signatures.

Each wrapper validates like the reference's TORCH_CHECKs (raising RuntimeError), allocates
outputs / workspace with the torch caching allocator, and enqueues the HIP kernels on the
current torch stream through the C ABI (``_lib``). There is no CPU fallback.

Reference signatures mirrored:
  attention_sparse_varlen, fused_offset_launch -> dyllm.attention_ops (attention.cpp:197-204)
  get_seqs_cuda, get_block_cuda, reset_full_cuda, reset_block_cuda, scatter_update_cuda
                                               -> dyllm.cache (cache.cpp:19-25)
  flash_attn_varlen_func                       -> flash-attn call sites attention.py:41-52, :76-87
  tensor_parallel_cosine_mask                  -> parallel_state.py:52-66
"""
from __future__ import annotations

import ctypes
import time

import torch

from . import _lib


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check(t, name, dtype=None, dim=None, device=None):
    if t is None:
        raise RuntimeError(f"{name} must be defined")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor")
    if device is not None and t.device != device:
        raise RuntimeError(f"{name} must be on {device}")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} has an invalid dtype ({t.dtype}, expected {dtype})")
    if dim is not None and t.dim() != dim:
        raise RuntimeError(f"{name} must be a {dim}D tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _i32(t):
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def _i64(t):
    return t if t.dtype == torch.int64 and t.is_contiguous() else t.to(torch.int64).contiguous()


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------
def attention_sparse_varlen(Q, K, V, C, o_sal, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                            total_seqlen, cu_salientlens, idx_salient_row, cosine_stats, cosine_out,
                            threshold=0.0, is_q_pruned=False, idx_salient_row_k=None, force_mask_v_rows=-1):
    """Column-sparse attention + stats + tau test (attention.cpp:64-179). Returns O = C +
    softmax(QK^T/sqrt(D)) V on non-salient rows and o_sal on salient rows; fills
    cosine_stats [T,3] and cosine_out [T] (bool). ``force_mask_v_rows`` is accepted for
    signature compatibility (the HIP kernel always skips salient-free key groups)."""
    dev = Q.device
    for t, n in ((Q, "Q"), (K, "K"), (V, "V"), (C, "C"), (o_sal, "o_sal")):
        _check(t, n, torch.bfloat16, 3, dev)
    for t, n in ((cu_seqlens_q, "cu_seqlens_q"), (cu_seqlens_k, "cu_seqlens_k"),
                 (cu_salientlens, "cu_salientlens"), (idx_salient_row, "idx_salient_row")):
        _check(t, n, torch.int32, 1, dev)
    _check(cosine_stats, "cosine_stats", torch.float32, 2, dev)
    _check(cosine_out, "cosine_out", torch.bool, 1, dev)
    if K.shape != V.shape:
        raise RuntimeError("K and V must have the same shape")
    if C.shape != Q.shape:
        raise RuntimeError("C must have the same shape as Q")
    if o_sal.shape[0] != idx_salient_row.numel() or o_sal.shape[1:] != Q.shape[1:]:
        raise RuntimeError("o_sal must be [idx_salient_row.numel(), Q.size(1), Q.size(2)]")
    if total_seqlen != Q.shape[0]:
        raise RuntimeError("total_seqlen must equal Q.size(0)")
    if tuple(cosine_stats.shape) != (Q.shape[0], 3):
        raise RuntimeError("cosine_stats must be [Q.size(0), 3]")
    if cosine_out.numel() != Q.shape[0]:
        raise RuntimeError("cosine_out must contain Q.size(0) elements")
    if not (cu_seqlens_q.numel() >= 2 and cu_seqlens_q.numel() == cu_seqlens_k.numel() == cu_salientlens.numel()):
        raise RuntimeError("cu_seqlens_q, cu_seqlens_k, and cu_salientlens must have the same B+1 length")
    if force_mask_v_rows not in (-1, 0, 1):
        raise RuntimeError("force_mask_v_rows must be -1, 0, or 1")
    idx_k = None
    if is_q_pruned:
        _check(idx_salient_row_k, "idx_salient_row_k", torch.int32, 1, dev)
        if idx_salient_row_k.numel() != idx_salient_row.numel():
            raise RuntimeError("parallel Q/K pruning requires matching salient Q and K index counts")
        idx_k = idx_salient_row_k
    B = cu_seqlens_q.numel() - 1
    H, D = Q.shape[1], Q.shape[2]
    O = torch.empty_like(Q)
    ws_bytes = _lib.load().dyllm_attention_sparse_workspace_bytes(B, H, Q.shape[0], int(max_seqlen_k))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("dyllm_attention_sparse_varlen", _ptr(Q), _ptr(K), _ptr(V), _ptr(C), _ptr(o_sal), _ptr(O), B, H,
              K.shape[1], D, _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), int(max_seqlen_q), int(max_seqlen_k),
              Q.shape[0], idx_salient_row.numel(), _ptr(cu_salientlens), _ptr(idx_salient_row), _ptr(idx_k),
              _ptr(cosine_stats), _ptr(cosine_out), float(threshold), _ptr(ws), ws_bytes, _stream())
    return O


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, q_rows=None, kv_start=None):
    """Non-causal varlen attention (the two flash_attn_varlen_func call sites). With
    ``q_rows`` (int32), compact row j of the output attends with q[q_rows[j]] and
    cu_seqlens_q is the prefix of the compact rows -- the row-sparse call
    ``flash_attn_varlen_func(q[idx], ...)`` without materialising q[idx]. With ``kv_start``
    (int64 [B]) sequence b's keys start at row kv_start[b] of k/v (a per-layer cache) instead
    of cu_seqlens_k[b]."""
    if causal or dropout_p != 0.0:
        raise RuntimeError("only non-causal attention without dropout is implemented")
    dev = q.device
    _check(q, "q", torch.bfloat16, 3, dev)
    _check(k, "k", torch.bfloat16, 3, dev)
    _check(v, "v", torch.bfloat16, 3, dev)
    cu_q, cu_k = _i32(cu_seqlens_q), _i32(cu_seqlens_k)
    D = q.shape[2]
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    if q_rows is not None:
        q_rows = _i32(q_rows)
        n_out = q_rows.numel()
    else:
        n_out = q.shape[0]
    o = torch.empty((n_out, q.shape[1], D), dtype=q.dtype, device=dev)
    if n_out == 0:
        return o
    _lib.call("dyllm_flash_attn_varlen", _ptr(q), _ptr(k), _ptr(v), _ptr(o), cu_q.numel() - 1, q.shape[1],
              k.shape[1], D, _ptr(cu_q), _ptr(cu_k), _ptr(kv_start), int(max_seqlen_q), int(max_seqlen_k),
              float(scale), _ptr(q_rows), _stream())
    return o


def attention_colsparse_cached(q, k_cache, kv_start, dv_compact, c_cache, c_start, o_sal, cu_seqlens_q,
                               cu_seqlens_k, max_seqlen_q, max_seqlen_k, total_k, idx_salient_q, idx_salient_k,
                               threshold, c_inplace=True, out=None, cosine_stats=None, cosine_out=None):
    """Column-sparse attention reading K and the context straight from the per-layer caches
    and a compact dV (rows follow idx_salient_k). Returns (O, stats [T,3], mask [T] bool);
    with ``c_inplace`` the new context rows are also written into ``c_cache``."""
    dev = q.device
    Tq, H, D = q.shape
    Hkv = k_cache.shape[1] if k_cache.dim() == 3 else k_cache.shape[1] // D
    B = cu_seqlens_q.numel() - 1
    n = idx_salient_q.numel()
    O = torch.empty_like(q) if out is None else out
    stats = torch.empty(Tq, 3, dtype=torch.float32, device=dev) if cosine_stats is None else cosine_stats
    mask = torch.empty(Tq, dtype=torch.bool, device=dev) if cosine_out is None else cosine_out
    ws_bytes = _lib.load().dyllm_attention_colsparse_workspace_bytes(B, H, Tq, int(total_k), int(max_seqlen_k))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.call("dyllm_attention_colsparse_cached", _ptr(q), _ptr(k_cache), _ptr(kv_start), _ptr(dv_compact),
              _ptr(c_cache), _ptr(c_start), int(bool(c_inplace)), _ptr(o_sal), _ptr(O), B, H, Hkv, D,
              _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), int(max_seqlen_q), int(max_seqlen_k), Tq, int(total_k), n,
              _ptr(idx_salient_q), _ptr(idx_salient_k), _ptr(stats), _ptr(mask), float(threshold), _ptr(ws),
              ws_bytes, _stream())
    return O, stats, mask


def v_delta_update(v_cache, v_new, dest_rows):
    """dv = v_new - v_cache[dest_rows]; v_cache[dest_rows] = v_new (attention.py:67-74)."""
    v_new = v_new.flatten(1).contiguous()
    dv = torch.empty_like(v_new)
    if v_new.shape[0]:
        _lib.call("dyllm_v_delta_update", _ptr(v_cache), _ptr(v_new), _ptr(dest_rows), v_new.shape[0],
                  v_new.shape[1], _ptr(dv), _stream())
    return dv


def seq_row_starts(seq_starts, seq_ids, cu_seqlens_k=None, cu_seqlens_q=None):
    """First cache row of each running sequence (+ the tail-block offset with cu_seqlens_q)."""
    out = torch.empty(seq_ids.numel(), dtype=torch.int64, device=seq_ids.device)
    _lib.call("dyllm_seq_row_starts", _ptr(seq_starts), _ptr(seq_ids), _ptr(cu_seqlens_k), _ptr(cu_seqlens_q),
              seq_ids.numel(), _ptr(out), _stream())
    return out


# ---------------------------------------------------------------------------------------
# saliency / compaction
# ---------------------------------------------------------------------------------------
def tensor_parallel_cosine_mask(stats, threshold):
    """cos < threshold from [T,3] fp32 stats (parallel_state.py:52-66, world size 1)."""
    _check(stats, "stats", torch.float32, 2)
    out = torch.empty(stats.shape[0], dtype=torch.bool, device=stats.device)
    _lib.call("dyllm_cosine_mask", _ptr(stats), stats.shape[0], float(threshold), _ptr(out), _stream())
    return out


def saliency_stats(c_new, c_old, threshold):
    """Standalone saliency pass over two bf16 row sets: ([T,3] fp32 stats, [T] bool mask)."""
    _check(c_new, "c_new", torch.bfloat16)
    _check(c_old, "c_old", torch.bfloat16)
    if c_new.shape != c_old.shape:
        raise RuntimeError("c_new and c_old must have the same shape")
    T = c_new.shape[0]
    D = c_new.numel() // max(T, 1)
    stats = torch.empty(T, 3, dtype=torch.float32, device=c_new.device)
    mask = torch.empty(T, dtype=torch.bool, device=c_new.device)
    _lib.call("dyllm_saliency_stats", _ptr(c_new), _ptr(c_old), T, D, float(threshold), _ptr(stats), _ptr(mask),
              _stream())
    return stats, mask


_HOST_META_TIMEOUT_S = 60.0
# count written by the step's compaction when its bounded look-back over the earlier workgroups'
# counts ran out (kCompactLookbackFailed in the library)
_COMPACT_LOOKBACK_FAILED = -2


def _check_count(n):
    if n == _COMPACT_LOOKBACK_FAILED:
        raise RuntimeError("salient compaction failed: a workgroup's look-back over the earlier counts did not "
                           "complete (the next salient set was not written)")
    return n


class Compacted:
    """Device results of one compaction; ``count`` stays on the device until asked for."""

    def __init__(self, idx64, idx32, idx_k, cu_salientlens, count, idx_k32=None, host_meta=None, dest_rows=None,
                 dest_starts=None):
        self.idx64, self.idx32, self.idx_k, self.idx_k32 = idx64, idx32, idx_k, idx_k32
        self.cu_salientlens, self.count = cu_salientlens, count
        self.host_meta = host_meta
        # rows of the salient set in the cache whose sequence-start table is dest_starts
        self.dest_rows, self.dest_starts = dest_rows, dest_starts

    def host(self):
        """(count, cu_salientlens as a list): one device->host read for both. When the producing
        kernel writes them into pinned host memory (host_meta, pre-filled with -1 before the
        launch; every entry is written once, by the block that owns it, and fenced to system
        scope), the host polls that buffer until no entry is negative: no event, no stream
        synchronisation, nothing enqueued between the kernel and the next launch."""
        if self.host_meta is not None:
            hm = self.host_meta
            deadline = None
            while True:
                h = hm.tolist()
                if min(h) >= 0 or h[0] == _COMPACT_LOOKBACK_FAILED:
                    break
                now = time.monotonic()
                if deadline is None:
                    deadline = now + _HOST_META_TIMEOUT_S
                elif now > deadline:
                    # the kernel did not run (an error earlier on the stream): surface it
                    if torch.cuda.is_available():
                        torch.cuda.synchronize()
                    raise RuntimeError("salient count was not written by the compaction kernel")
        else:
            h = torch.cat([self.count, self.cu_salientlens]).cpu().tolist()
        _check_count(h[0])
        return h[0], h[1:]

    def n(self) -> int:
        return _check_count(int(self.count.item()))

    def trimmed(self):
        n = self.n()
        return (self.idx64[:n], self.idx32[:n], None if self.idx_k is None else self.idx_k[:n],
                self.cu_salientlens)


def salient_compact(mask, cu_seqlens_q, cu_promptlens=None):
    """torch.nonzero(mask) + searchsorted(idxs, cu_seqlens_q) + fused_offset, on the device
    (attention.py:147-166). Index buffers are capacity-sized; see ``Compacted``."""
    dev = mask.device
    _check(mask, "mask", None, 1, dev)
    if mask.dtype not in (torch.bool, torch.uint8):
        raise RuntimeError("mask must be bool or uint8")
    T = mask.numel()
    cu_q = _i32(cu_seqlens_q)
    B = cu_q.numel() - 1
    idx64 = torch.empty(max(T, 1), dtype=torch.int64, device=dev)
    idx32 = torch.empty(max(T, 1), dtype=torch.int32, device=dev)
    idx_k = torch.empty(max(T, 1), dtype=torch.int64, device=dev) if cu_promptlens is not None else None
    cu_p = _i32(cu_promptlens) if cu_promptlens is not None else None
    cu_sal = torch.empty(B + 1, dtype=torch.int32, device=dev)
    count = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("dyllm_salient_compact", _ptr(mask), T, _ptr(cu_q), B, _ptr(cu_p), _ptr(idx64), _ptr(idx32),
              _ptr(idx_k), _ptr(cu_sal), _ptr(count), _stream())
    return Compacted(idx64, idx32, idx_k, cu_sal, count)


class StepBuffers:
    """Reusable outputs and workspace of ``sparse_attention_step`` for one layer and shape."""

    def __init__(self, key, dev, Tq, Tk, B, H, Hkv, D, max_k, q_pruned):
        self.key = key
        i64, i32 = dict(dtype=torch.int64, device=dev), dict(dtype=torch.int32, device=dev)
        self.out = torch.empty((Tq, H, D), dtype=torch.bfloat16, device=dev)
        self.stats = torch.empty((Tq, 3), dtype=torch.float32, device=dev)
        self.mask = torch.empty(Tq, dtype=torch.bool, device=dev)
        self.idx64 = torch.empty(max(Tq, 1), **i64)
        self.idx32 = torch.empty(max(Tq, 1), **i32)
        self.idx_k64 = torch.empty(max(Tq, 1), **i64) if q_pruned else None
        self.idx_k32 = torch.empty(max(Tq, 1), **i32) if q_pruned else None
        self.meta = torch.empty(B + 2, **i32)          # [count, cu_salientlens...]
        self.count, self.cu_sal = self.meta[0:1], self.meta[1:]
        self.host_meta = torch.empty(B + 2, dtype=torch.int32, pin_memory=True)
        self.dest_rows = torch.empty(max(Tq, 1), **i64)
        self.dest_starts = None       # the cache table dest_rows was computed for, in the last call
        self.ws_bytes = _lib.load().dyllm_sparse_step_workspace_bytes(B, H, Hkv, D, Tq, Tk, max_k, Tq)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=dev)

    def compacted(self):
        return Compacted(self.idx64, self.idx32, self.idx_k64, self.cu_sal, self.count, self.idx_k32,
                         self.host_meta, self.dest_rows if self.dest_starts is not None else None, self.dest_starts)


class KvRows:
    """The salient-row K/V projection output, handed to ``Attention.forward`` in place of ``v``
    (llada.py:108-147): its epilogue -- optional k_norm, neox RoPE, the K-cache row write
    (CacheManager.scatter_update) -- and the v rows are consumed by the sparse step's first launch
    (dyllm_sparse_attention_step_kv), so no compact v or separate scatter pass is needed.

    kv: [rows, >= 2 * num_kv_heads * 128] bf16 = [k | v]; row j of the salient list reads row
    kv_rows[j] (None: j); positions[pos_idx[j]] (None: positions[j]) is its rotary position;
    k_cache / k_seq_starts: the K cache slab and its per-sequence-id first rows."""

    def __init__(self, kv, num_kv_heads, positions, cos, sin, k_cache, k_seq_starts, kv_rows=None, pos_idx=None,
                 k_norm_weight=None, eps=1e-6):
        _check(kv, "kv", torch.bfloat16, 2)
        kv_size = num_kv_heads * 128
        if kv.shape[1] < 2 * kv_size or kv.stride(1) != 1 or kv.stride(0) % 8:
            raise RuntimeError("kv rows must hold k then v (2 * num_kv_heads * 128 contiguous values, 16-byte rows)")
        for t, n in ((cos, "cos"), (sin, "sin")):
            _check(t, n, torch.float32, 2)
            if t.shape[1] != 64 or not t.is_contiguous():
                raise RuntimeError(f"{n} must be a contiguous [max_position, 64] fp32 table")
        if cos.shape != sin.shape:
            raise RuntimeError("cos and sin tables must have the same shape")
        if k_cache.dtype != torch.bfloat16 or k_cache.dim() != 2 or k_cache.shape[1] != kv_size:
            raise RuntimeError("k_cache must be bf16 [rows, num_kv_heads * 128]")
        if k_norm_weight is not None:
            _check(k_norm_weight, "k_norm_weight", torch.bfloat16, 1)
            if k_norm_weight.numel() != 128:
                raise RuntimeError("k_norm_weight must have head_dim (128) entries")
        self.kv, self.num_kv_heads = kv, num_kv_heads
        self.positions = _i64(positions)
        self.cos, self.sin = cos, sin
        self.k_cache, self.k_seq_starts = k_cache, k_seq_starts
        self.kv_rows = None if kv_rows is None else _i32(kv_rows)
        self.pos_idx = None if pos_idx is None else _i32(pos_idx)
        self.k_norm_weight, self.eps = k_norm_weight, float(eps)

    def struct(self):
        e = _lib.KvEpilogue()
        e.kv, e.ld_kv, e.kv_rows = _ptr(self.kv), self.kv.stride(0), _ptr(self.kv_rows)
        e.positions, e.pos_idx = _ptr(self.positions), _ptr(self.pos_idx)
        e.cos_table, e.sin_table, e.max_position = _ptr(self.cos), _ptr(self.sin), self.cos.shape[0]
        e.k_norm_weight, e.eps = _ptr(self.k_norm_weight), self.eps
        e.k_cache, e.k_seq_starts = _ptr(self.k_cache), _ptr(self.k_seq_starts)
        return e


def sparse_attention_step(bufs, q, k, v_cache, v_seq_starts, v_new, c_cache, c_seq_starts, seq_ids, cu_seqlens_q,
                          cu_seqlens_k, cu_promptlens, max_seqlen_q, max_seqlen_k, total_k, n_sal, max_salientlen,
                          cu_salientlens, idx_q32, idx_k64, idx_k32, softmax_scale, threshold, k_start=None,
                          dest_seq_starts=None):
    """The sparse branch of Attention.forward in one native call (dyllm_sparse_attention_step).
    Results land in ``bufs`` (out / stats / mask and the next salient set, left on the device);
    with ``dest_seq_starts`` (another per-layer cache's start table) also the rows of the next
    salient set in that cache (``bufs.dest_rows``). ``v_new`` may be a ``KvRows`` (then ``k`` and
    ``k_start`` are None: K is read from its cache after the epilogue, through
    dyllm_sparse_attention_step_kv)."""
    Tq, H, D = q.shape
    bufs.host_meta.fill_(-1)   # "not written yet" for Compacted.host()
    bufs.dest_starts = dest_seq_starts
    if isinstance(v_new, KvRows):
        if k is not None or k_start is not None:
            raise RuntimeError("with KvRows, K comes from the K cache: k and k_start must be None")
        epi = v_new.struct()
        head = ("dyllm_sparse_attention_step_kv", ctypes.addressof(epi), _ptr(q), None, None)
        Hkv, v_new = v_new.num_kv_heads, None
    else:
        head = ("dyllm_sparse_attention_step", _ptr(q), _ptr(k), _ptr(k_start))
        Hkv = v_new.shape[1] if v_new.dim() == 3 else v_cache.shape[1] // D
    _lib.call(*head, _ptr(v_cache), _ptr(v_seq_starts),
              _ptr(v_new), _ptr(c_cache), _ptr(c_seq_starts), _ptr(seq_ids), seq_ids.numel(), H, Hkv, D,
              _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), _ptr(cu_promptlens), int(max_seqlen_q), int(max_seqlen_k), Tq,
              int(total_k), int(n_sal), int(max_salientlen), _ptr(cu_salientlens), _ptr(idx_q32), _ptr(idx_k64),
              _ptr(idx_k32), float(softmax_scale), float(threshold), _ptr(bufs.out), _ptr(bufs.stats),
              _ptr(bufs.mask), _ptr(bufs.idx64), _ptr(bufs.idx32), _ptr(bufs.idx_k64), _ptr(bufs.idx_k32),
              _ptr(bufs.cu_sal), _ptr(bufs.count), _ptr(dest_seq_starts),
              _ptr(bufs.dest_rows if dest_seq_starts is not None else None), _ptr(bufs.host_meta), _ptr(bufs.ws),
              bufs.ws_bytes, _stream())
    return bufs


def sparse_attention_step_noalloc(bufs, q, k, v_cache, v_seq_starts, v_new, c_cache, c_seq_starts, seq_ids,
                                  cu_seqlens_q, cu_seqlens_k, cu_promptlens, max_seqlen_q, max_seqlen_k, total_k,
                                  n_sal, max_salientlen, cu_salientlens, idx_q32, idx_k64, idx_k32, softmax_scale,
                                  threshold, k_start=None, dest_seq_starts=None):
    """``sparse_attention_step`` through dyllm_sparse_attention_step_noalloc: the workspace is the
    library's own per-GPU scratch array (``bufs.ws`` is not used), so the call allocates nothing."""
    Tq, H, D = q.shape
    Hkv = v_new.shape[1] if v_new.dim() == 3 else v_cache.shape[1] // D
    bufs.host_meta.fill_(-1)
    bufs.dest_starts = dest_seq_starts
    _lib.call("dyllm_sparse_attention_step_noalloc", _ptr(q), _ptr(k), _ptr(k_start), _ptr(v_cache),
              _ptr(v_seq_starts), _ptr(v_new), _ptr(c_cache), _ptr(c_seq_starts), _ptr(seq_ids), seq_ids.numel(), H,
              Hkv, D, _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), _ptr(cu_promptlens), int(max_seqlen_q),
              int(max_seqlen_k), Tq, int(total_k), int(n_sal), int(max_salientlen), _ptr(cu_salientlens),
              _ptr(idx_q32), _ptr(idx_k64), _ptr(idx_k32), float(softmax_scale), float(threshold), _ptr(bufs.out),
              _ptr(bufs.stats), _ptr(bufs.mask), _ptr(bufs.idx64), _ptr(bufs.idx32), _ptr(bufs.idx_k64),
              _ptr(bufs.idx_k32), _ptr(bufs.cu_sal), _ptr(bufs.count), _ptr(dest_seq_starts),
              _ptr(bufs.dest_rows if dest_seq_starts is not None else None), _ptr(bufs.host_meta), _stream())
    return bufs


def attention_kernel_info(dim, mask_v_rows=False):
    """attention.cpp:205-208: launch resources of this build's main attention kernel,
    [regs, local_bytes, static_smem, dynamic_smem, tb_size, max_active_blocks_per_sm, block_q,
    block_k, d_split, ok] (per CU on this GPU)."""
    out = (ctypes.c_int64 * 10)()
    _lib.call("dyllm_attention_kernel_info", int(dim), int(bool(mask_v_rows)), ctypes.addressof(out))
    return list(out)


def fused_offset_launch(idxs, num_idxs, cu_promptlens, cu_salientlens, out_tensor, max_threads):
    """attention_aux_kernels.cu:173-200 (same argument checks)."""
    dev = idxs.device
    for t, n in ((idxs, "idxs"), (num_idxs, "num_idxs"), (cu_promptlens, "cu_promptlens"),
                 (cu_salientlens, "cu_salientlens")):
        _check(t, n, torch.int32, 1, dev)
    if num_idxs.numel() != 1:
        raise RuntimeError("num_idxs must contain exactly one element")
    if cu_promptlens.numel() != cu_salientlens.numel():
        raise RuntimeError("cu_promptlens and cu_salientlens must have the same length")
    _check(out_tensor, "out_tensor", torch.int64, 1, dev)
    if not (0 <= max_threads <= out_tensor.numel()):
        raise RuntimeError("max_threads must fit out_tensor")
    if max_threads == 0:
        return
    _lib.call("dyllm_fused_offset_launch", _ptr(idxs), _ptr(num_idxs), _ptr(cu_promptlens), _ptr(cu_salientlens),
              cu_promptlens.numel() - 1, _ptr(out_tensor), int(max_threads), _stream())


# ---------------------------------------------------------------------------------------
# packed row caches (dyllm.cache)
# ---------------------------------------------------------------------------------------
def _row_bytes(t):
    return t.shape[1] * t.element_size()


def _check_cache(cache, seq_starts, seq_ids):
    _check(cache, "cache", None, 2)
    _check(seq_starts, "seq_starts", torch.int64, 1)
    _check(seq_ids, "seq_ids", torch.int64, 1)
    if (cache.shape[1] * cache.element_size()) % 16 != 0:
        raise RuntimeError("row size must be a multiple of 16 bytes (D % 8 == 0 for bf16)")


def get_seqs_cuda(cache, seq_starts, cu_seqlens, seq_ids, total_seqlen):
    _check_cache(cache, seq_starts, seq_ids)
    cu = _i32(cu_seqlens)
    out = torch.empty((int(total_seqlen), cache.shape[1]), dtype=cache.dtype, device=cache.device)
    _lib.call("dyllm_get_seqs", _ptr(cache), _ptr(out), _row_bytes(cache), _ptr(seq_starts), _ptr(cu),
              _ptr(seq_ids), seq_ids.numel(), int(total_seqlen), _stream())
    return out


def get_block_cuda(cache, seq_starts, cu_seqlens, cu_seqlens_q, seq_ids, total_seqlen):
    _check_cache(cache, seq_starts, seq_ids)
    cu, cq = _i32(cu_seqlens), _i32(cu_seqlens_q)
    out = torch.empty((int(total_seqlen), cache.shape[1]), dtype=cache.dtype, device=cache.device)
    _lib.call("dyllm_get_block", _ptr(cache), _ptr(out), _row_bytes(cache), _ptr(seq_starts), _ptr(cu), _ptr(cq),
              _ptr(seq_ids), seq_ids.numel(), int(total_seqlen), _stream())
    return out


def reset_full_cuda(cache, inp, seq_starts, cu_seqlens, seq_ids, total_seqlen):
    _check_cache(cache, seq_starts, seq_ids)
    _check(inp, "in", cache.dtype, 2)
    cu = _i32(cu_seqlens)
    _lib.call("dyllm_reset_full", _ptr(cache), _ptr(inp), _row_bytes(cache), _ptr(seq_starts), _ptr(cu),
              _ptr(seq_ids), seq_ids.numel(), int(total_seqlen), _stream())


def reset_block_cuda(cache, inp, seq_starts, cu_seqlens, cu_seqlens_q, seq_ids, total_seqlen):
    _check_cache(cache, seq_starts, seq_ids)
    _check(inp, "in", cache.dtype, 2)
    cu, cq = _i32(cu_seqlens), _i32(cu_seqlens_q)
    _lib.call("dyllm_reset_block", _ptr(cache), _ptr(inp), _row_bytes(cache), _ptr(seq_starts), _ptr(cu), _ptr(cq),
              _ptr(seq_ids), seq_ids.numel(), int(total_seqlen), _stream())


def scatter_update_cuda(cache, new_vals, row_idx, cu_seqlens, seq_starts, seq_ids):
    _check_cache(cache, seq_starts, seq_ids)
    new_vals = new_vals.flatten(1).contiguous()
    _check(new_vals, "new_vals", cache.dtype, 2)
    if new_vals.shape[1] != cache.shape[1]:
        raise RuntimeError("new_vals row width must match the cache")
    ri = _i64(row_idx)
    if ri.numel() != new_vals.shape[0]:
        raise RuntimeError("row_idx must have one entry per new row")
    if ri.numel() == 0:
        return
    cu = _i32(cu_seqlens)
    _lib.call("dyllm_scatter_update", _ptr(cache), _ptr(new_vals), _row_bytes(cache), _ptr(ri), ri.numel(),
              _ptr(cu), _ptr(seq_starts), _ptr(seq_ids), seq_ids.numel(), _stream())


def scatter_dest_rows(row_idx, cu_seqlens, seq_starts, seq_ids, count=None):
    """Cache rows of packed row indices; with ``count`` (device int32 [1]) only the first
    count[0] entries of the capacity-sized ``row_idx`` are mapped."""
    ri = _i64(row_idx)
    cu = _i32(cu_seqlens)
    dest = torch.empty_like(ri)
    if ri.numel():
        _lib.call("dyllm_scatter_dest_rows", _ptr(ri), ri.numel(), _ptr(count), _ptr(cu), _ptr(seq_starts),
                  _ptr(seq_ids), seq_ids.numel(), _ptr(dest), _stream())
    return dest


def gather_rows_2D(x, row_idx):
    """utils/util.py:19-36: x[row_idx] for a [L, D] tensor."""
    _check(x, "x", None, 2)
    ri = _i64(row_idx)
    out = torch.empty((ri.numel(), x.shape[1]), dtype=x.dtype, device=x.device)
    if ri.numel():
        _lib.call("dyllm_gather_rows", _ptr(x), x.shape[0], _ptr(out), _row_bytes(x), _ptr(ri), ri.numel(), _stream())
    return out


# ---------------------------------------------------------------------------------------
# FFN / MoE
# ---------------------------------------------------------------------------------------
def _gemm_source(x, name="x"):
    """The GEMM kernels address an operand with 32-bit byte offsets: a gathered input must span
    less than 4 GiB (the library cannot see a gathered source's extent)."""
    if x.shape[0] and ((x.shape[0] - 1) * x.stride(0) + x.shape[1]) * 2 > (1 << 32):
        raise ValueError(f"{name} spans more than 4 GiB; the GEMM kernels address it with 32-bit offsets")


def ffn_gate_up(x, w_gate_up, rows_idx=None, count=None, hint=0):
    """h = silu(a Wg^T) * (a Wu^T) for a = x[rows_idx] (gathered inside the GEMM). With
    ``count`` (device int32 [1]) ``rows_idx`` is a capacity-sized buffer of which the first
    count[0] rows are used -- no host synchronisation; ``hint`` is the expected count."""
    _check(x, "x", torch.bfloat16, 2)
    _gemm_source(x)
    _check(w_gate_up, "w_gate_up", torch.bfloat16, 2)
    hidden = x.shape[1]
    inter = w_gate_up.shape[0] // 2
    if w_gate_up.shape[1] != hidden:
        raise RuntimeError("w_gate_up must be [2I, hidden]")
    ri = _i32(rows_idx) if rows_idx is not None else None
    M = ri.numel() if ri is not None else x.shape[0]
    h = torch.empty((M, inter), dtype=x.dtype, device=x.device)
    if M:
        _lib.call("dyllm_ffn_gate_up", _ptr(x), x.stride(0), _ptr(ri), M, _ptr(count), int(hint), _ptr(w_gate_up),
                  hidden, inter, _ptr(h), _stream())
    return h


def ffn_down(h, w_down, out=None, out_rows=None, count=None, hint=0):
    """y = h Wd^T, written to out[out_rows[m]] when given (in-place scatter) else a new tensor;
    ``count``/``hint`` as for ffn_gate_up."""
    _check(h, "h", torch.bfloat16, 2)
    _check(w_down, "w_down", torch.bfloat16, 2)
    M, inter = h.shape
    hidden = w_down.shape[0]
    if w_down.shape[1] != inter:
        raise RuntimeError("w_down must be [hidden, I]")
    if out is None:
        out = torch.empty((M, hidden), dtype=h.dtype, device=h.device)
        orow = None
    else:
        _check(out, "out", torch.bfloat16, 2)
        orow = _i64(out_rows) if out_rows is not None else None
    if M:
        ws_bytes = _lib.load().dyllm_ffn_down_workspace_bytes(M, int(hint), hidden, inter)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
        _lib.call("dyllm_ffn_down", _ptr(h), M, _ptr(count), int(hint), _ptr(w_down), hidden, inter, _ptr(out),
                  _ptr(orow), _ptr(ws), ws_bytes, _stream())
    return out


def linear(x, w, bias=None, rows_idx=None, count=None, hint=0):
    """F.linear(x[rows_idx], w, bias) as one gathered GEMM (dyllm_linear): the salient-row
    kv_proj of llada.py:108 / dream.py:103 / lladamoe.py:204. ``count``/``hint`` as for
    ffn_gate_up (rows beyond count[0] are left unwritten)."""
    _check(x, "x", torch.bfloat16, 2)
    _gemm_source(x)
    _check(w, "w", torch.bfloat16, 2)
    n_out, k_in = w.shape
    if x.shape[1] != k_in:
        raise RuntimeError("x must be [rows, in_features] with in_features = w.shape[1]")
    if x.stride(1) != 1:
        raise RuntimeError("x rows must be contiguous")
    if bias is not None:
        _check(bias, "bias", torch.bfloat16, 1)
        if bias.numel() != n_out or not bias.is_contiguous():
            raise RuntimeError("bias must be a contiguous [out_features] tensor")
    ri = _i32(rows_idx) if rows_idx is not None else None
    M = ri.numel() if ri is not None else x.shape[0]
    out = torch.empty((M, n_out), dtype=x.dtype, device=x.device)
    if M:
        ws_bytes = _lib.load().dyllm_linear_workspace_bytes(M, int(hint), n_out, k_in)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        _lib.call("dyllm_linear", _ptr(x), x.stride(0), _ptr(ri), M, _ptr(count), int(hint), _ptr(w), n_out, k_in,
                  _ptr(bias), _ptr(out), _ptr(ws), ws_bytes, _stream())
    return out


def rope_(x, num_heads, positions, cos, sin, norm_weight=None, eps=1e-6):
    """In-place neox RoPE of x [rows, num_heads * 128] at positions[row] (rotary_embedding.py:8-16,
    47-54), after an optional per-head RMSNorm with norm_weight (q_norm, layernorm.py:15-24)
    (dyllm_rope). x may be a row-strided view (the k half of a [k | v] projection). Returns x."""
    if x is None or not x.is_cuda or x.dtype != torch.bfloat16 or x.dim() != 2:
        raise RuntimeError("x must be a bf16 2D GPU tensor")
    _check(positions, "positions", None, 1)
    positions = _i64(positions)
    for t, n in ((cos, "cos"), (sin, "sin")):
        _check(t, n, torch.float32, 2)
        if t.shape[1] != 64 or not t.is_contiguous():
            raise RuntimeError(f"{n} must be a contiguous [max_position, 64] fp32 table")
    if x.shape[1] != num_heads * 128 or x.stride(1) != 1:
        raise RuntimeError("x must be [rows, num_heads * 128] with contiguous rows")
    if positions.numel() < x.shape[0]:
        raise RuntimeError("positions must have one entry per row")
    if norm_weight is not None:
        _check(norm_weight, "norm_weight", torch.bfloat16, 1)
        if norm_weight.numel() != 128:
            raise RuntimeError("norm_weight must have head_dim (128) entries")
    if x.shape[0]:
        _lib.call("dyllm_rope", _ptr(x), x.stride(0), x.shape[0], num_heads, 128, _ptr(positions), _ptr(cos),
                  _ptr(sin), cos.shape[0], _ptr(norm_weight), float(eps), _stream())
    return x


def kv_rope_scatter(kv, num_kv_heads, positions, cos, sin, k_cache, k_rows, cu_seqlens_k, seq_starts, seq_ids,
                    pos_idx=None, k_norm_weight=None, eps=1e-6, count=None):
    """K/V epilogue of the salient-row projection (dyllm_kv_rope_scatter): for each row j of
    kv = [k | v], k -> (per-head RMSNorm with k_norm_weight) -> neox RoPE at
    positions[pos_idx[j] or j] -> K-cache row of packed K row k_rows[j]; returns v
    [rows, Hkv, 128] (the sparse step's v_new). cos / sin: fp32 [max_position, 64]."""
    _check(kv, "kv", torch.bfloat16, 2)
    _check_cache(k_cache, seq_starts, seq_ids)
    _check(positions, "positions", None, 1)
    positions = _i64(positions)
    for t, n in ((cos, "cos"), (sin, "sin")):
        _check(t, n, torch.float32, 2)
        if t.shape[1] != 64 or not t.is_contiguous():
            raise RuntimeError(f"{n} must be a contiguous [max_position, 64] fp32 table")
    if cos.shape != sin.shape:
        raise RuntimeError("cos and sin tables must have the same shape")
    kv_size = num_kv_heads * 128
    if kv.shape[1] < 2 * kv_size or kv.stride(1) != 1:
        raise RuntimeError("kv rows must hold k then v (2 * num_kv_heads * 128 contiguous values)")
    if k_cache.shape[1] != kv_size or k_cache.dtype != torch.bfloat16:
        raise RuntimeError("k_cache must be bf16 [rows, num_kv_heads * 128]")
    if k_norm_weight is not None:
        _check(k_norm_weight, "k_norm_weight", torch.bfloat16, 1)
        if k_norm_weight.numel() != 128:
            raise RuntimeError("k_norm_weight must have head_dim (128) entries")
    rows = kv.shape[0]
    kr = _i64(k_rows)
    if kr.numel() < rows:
        raise RuntimeError("k_rows must have one entry per kv row")
    pi = _i32(pos_idx) if pos_idx is not None else None
    if pi is not None and pi.numel() < rows:
        raise RuntimeError("pos_idx must have one entry per kv row")
    v_out = torch.empty((rows, num_kv_heads, 128), dtype=kv.dtype, device=kv.device)
    if rows:
        _lib.call("dyllm_kv_rope_scatter", _ptr(kv), kv.stride(0), rows, _ptr(count), _ptr(pi), _ptr(positions),
                  _ptr(cos), _ptr(sin), cos.shape[0], num_kv_heads, 128, _ptr(k_norm_weight), float(eps),
                  _ptr(k_cache), _ptr(kr), _ptr(_i32(cu_seqlens_k)), _ptr(seq_starts), _ptr(seq_ids),
                  seq_ids.numel(), _ptr(v_out), _stream())
    return v_out


class CacheRows:
    """The queried rows of a per-layer row cache, not copied out: packed row r of sequence b reads
    slab row seq_starts[seq_ids[b]] + (Lk_b - Lq_b) + (r - cu_q[b]) (get_block addressing). The
    consumer (``rms_norm``) reads them in place; ``materialize()`` makes the packed copy."""

    def __init__(self, slab, seq_starts, seq_ids, cu_seqlens_k, cu_seqlens_q, rows):
        self.slab, self.seq_starts, self.seq_ids = slab, seq_starts, seq_ids
        self.cu_k, self.cu_q = _i32(cu_seqlens_k), _i32(cu_seqlens_q)
        self.rows = int(rows)
        self.shape = (self.rows, slab.shape[1])
        self.dtype, self.device = slab.dtype, slab.device

    def materialize(self):
        return get_block_cuda(self.slab, self.seq_starts, self.cu_k, self.cu_q, self.seq_ids, self.rows)


def rms_norm(x, weight, eps, residual=None, out=None, residual_out=None):
    """RMSNorm (layernorm.py:15-24) or, with ``residual``, the fused add + RMSNorm
    (layernorm.py:29-37) in one pass per row (dyllm_rms_norm). Returns y, or (y, residual_out)
    with residual_out = bf16(x + residual); ``out`` / ``residual_out`` may be x / residual
    (in place). ``x`` may be a ``CacheRows`` (rows read from the cache in place)."""
    if isinstance(x, CacheRows):
        return _rms_norm_cache_rows(x, weight, eps, residual, out, residual_out)
    _check(x, "x", torch.bfloat16, 2)
    _check(weight, "weight", torch.bfloat16, 1)
    rows, hidden = x.shape
    if weight.numel() != hidden or not weight.is_contiguous():
        raise RuntimeError("weight must be a contiguous [hidden] tensor")
    if x.stride(1) != 1:
        raise RuntimeError("x rows must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    _check(out, "out", torch.bfloat16, 2)
    if residual is not None:
        _check(residual, "residual", torch.bfloat16, 2)
        if residual.shape != x.shape or residual.stride(1) != 1:
            raise RuntimeError("residual must match x with contiguous rows")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    if rows:
        _lib.call("dyllm_rms_norm", _ptr(x), x.stride(0), _ptr(residual),
                  residual.stride(0) if residual is not None else 0, _ptr(weight), rows, hidden, float(eps),
                  _ptr(out), out.stride(0), _ptr(residual_out),
                  residual_out.stride(0) if residual_out is not None else 0, _stream())
    return out if residual is None else (out, residual_out)


def _rms_norm_cache_rows(x, weight, eps, residual, out, residual_out):
    _check(weight, "weight", torch.bfloat16, 1)
    rows, hidden = x.shape
    if weight.numel() != hidden or not weight.is_contiguous():
        raise RuntimeError("weight must be a contiguous [hidden] tensor")
    if x.slab.stride(1) != 1:
        raise RuntimeError("cache rows must be contiguous")
    if out is None:
        out = torch.empty(rows, hidden, dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16, 2)
    if residual is not None:
        _check(residual, "residual", torch.bfloat16, 2)
        if tuple(residual.shape) != (rows, hidden) or residual.stride(1) != 1:
            raise RuntimeError("residual must be [rows, hidden] with contiguous rows")
        if residual_out is None:
            residual_out = torch.empty_like(residual)
    if rows:
        _lib.call("dyllm_rms_norm_cache_rows", _ptr(x.slab), x.slab.stride(0), _ptr(x.seq_starts), _ptr(x.seq_ids),
                  _ptr(x.cu_k), _ptr(x.cu_q), x.cu_q.numel() - 1, _ptr(residual),
                  residual.stride(0) if residual is not None else 0, _ptr(weight), rows, hidden, float(eps),
                  _ptr(out), out.stride(0), _ptr(residual_out),
                  residual_out.stride(0) if residual_out is not None else 0, _stream())
    return out if residual is None else (out, residual_out)


# Row count from which the dense FFN of all rows (the full step) runs the library GEMMs around
# dyllm_silu_and_mul instead of the fused gate_up / down kernels: measured faster from 2048 rows on
# (LLaDA-8B shapes), where the fused GEMMs' gather and scatter epilogues have nothing to save.
DENSE_FFN_LIBRARY_ROWS = 2048


def silu_and_mul(gate_up, out=None):
    """SiluAndMul (activations.py:11-14) of a merged gate_up product [rows, 2I] (gate columns
    first): bf16(silu(g) * u) computed in fp32 with one rounding (dyllm_silu_and_mul)."""
    _check(gate_up, "gate_up", torch.bfloat16, 2)
    if gate_up.stride(1) != 1 or gate_up.shape[1] % 2:
        raise RuntimeError("gate_up must be [rows, 2I] with contiguous rows")
    rows, inter = gate_up.shape[0], gate_up.shape[1] // 2
    if out is None:
        out = torch.empty((rows, inter), dtype=gate_up.dtype, device=gate_up.device)
    else:
        _check(out, "out", torch.bfloat16, 2)
        if out.shape[0] < rows or out.shape[1] < inter or out.stride(1) != 1:
            raise RuntimeError("out must hold [rows, I] with contiguous rows")
    if rows:
        _lib.call("dyllm_silu_and_mul", _ptr(gate_up), gate_up.stride(0), rows, inter, _ptr(out), out.stride(0),
                  _stream())
    return out


def swiglu_ffn(x, w_gate_up, w_down, rows_idx=None, out=None, out_rows=None):
    """down(silu(a Wg^T) * (a Wu^T)) for a = x[rows_idx] (or all rows of x). With
    ``out``/``out_rows`` the result rows are written to out[out_rows[m]] (in-place scatter
    into a cache); otherwise a new [M, hidden] tensor is returned. A dense product of at least
    DENSE_FFN_LIBRARY_ROWS rows runs gate_up and down as library GEMMs around silu_and_mul (the
    same rounding points: g and u in bf16, silu(g) * u in fp32, h in bf16)."""
    _check(w_down, "w_down", torch.bfloat16, 2)
    if tuple(w_down.shape) != (x.shape[1], w_gate_up.shape[0] // 2):
        raise RuntimeError("weights must be w_gate_up [2I, hidden] and w_down [hidden, I]")
    if rows_idx is None and out is None and x.shape[0] >= DENSE_FFN_LIBRARY_ROWS:
        _check(x, "x", torch.bfloat16, 2)
        _check(w_gate_up, "w_gate_up", torch.bfloat16, 2)
        return torch.nn.functional.linear(silu_and_mul(torch.nn.functional.linear(x, w_gate_up)), w_down)
    h = ffn_gate_up(x, w_gate_up, rows_idx)
    return ffn_down(h, w_down, out, out_rows)


def moe_gate(hidden_states, router_weight, top_k, renormalize=False, rows_idx=None):
    """fp32 softmax top-k routing (fused_moe.py:375-408 without the DiffusionGemma extras); with
    ``rows_idx`` the tokens are rows rows_idx[t] of ``hidden_states``."""
    _check(hidden_states, "hidden_states", torch.bfloat16, 2)
    if hidden_states.stride(1) != 1 or hidden_states.stride(0) != hidden_states.shape[1]:
        raise RuntimeError("hidden_states must be contiguous")
    rw = router_weight.to(torch.bfloat16).contiguous()
    ri = _i32(rows_idx) if rows_idx is not None else None
    T = ri.numel() if ri is not None else hidden_states.shape[0]
    w = torch.empty((T, top_k), dtype=torch.bfloat16, device=hidden_states.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=hidden_states.device)
    if T:
        _lib.call("dyllm_moe_gate", _ptr(hidden_states), _ptr(ri), T, hidden_states.shape[1], _ptr(rw), rw.shape[0],
                  int(top_k), int(bool(renormalize)), _ptr(w), _ptr(ids), _stream())
    return w, ids


def moe_align_block_size(topk_ids, block_size, num_experts):
    """Device moe_align_block_size (fused_moe.py:37-85). Returns (sorted_token_ids,
    expert_ids, num_tokens_post_pad) with capacity-sized id buffers."""
    ids = _i32(topk_ids).reshape(-1)
    S = ids.numel()
    cap = -(-(S + num_experts * (block_size - 1)) // block_size) * block_size
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=ids.device)
    tile_e = torch.empty(cap // block_size, dtype=torch.int32, device=ids.device)
    npp = torch.empty(1, dtype=torch.int32, device=ids.device)
    _lib.call("dyllm_moe_align_block_size", _ptr(ids), S, num_experts, block_size, _ptr(sorted_ids), cap,
              _ptr(tile_e), _ptr(npp), _stream())
    return sorted_ids, tile_e, npp


def fused_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation="silu", out=None, out_rows=None,
                  rows_idx=None):
    """fused_experts (fused_moe.py:269-335) with SiLU gating. With ``rows_idx`` token t is row
    rows_idx[t] of ``hidden_states`` (the salient rows, gathered inside the first grouped GEMM)."""
    if activation != "silu":
        raise RuntimeError("only the silu activation (LLaDA-MoE) is implemented")
    x = hidden_states
    _check(x, "hidden_states", torch.bfloat16, 2)
    _check(w1, "w1", torch.bfloat16, 3)
    _check(w2, "w2", torch.bfloat16, 3)
    ri = None
    if rows_idx is not None:
        _gemm_source(x)
        ri = _i32(rows_idx)
        if ri.numel() != topk_ids.shape[0]:
            raise RuntimeError("rows_idx must have one entry per routed token")
        if x.stride(1) != 1 or x.stride(0) != x.shape[1]:
            raise RuntimeError("hidden_states must be contiguous when rows are gathered")
    T, hidden = (topk_ids.shape[0], x.shape[1]) if ri is not None else x.shape
    E, two_i, _ = w1.shape
    inter = two_i // 2
    top_k = topk_ids.shape[1]
    tw = topk_weights.to(torch.bfloat16).contiguous()
    ti = _i32(topk_ids)
    if out is None:
        out = torch.empty((T, hidden), dtype=x.dtype, device=x.device)
        orow = None
    else:
        orow = _i64(out_rows) if out_rows is not None else None
    if T == 0:
        return out
    ws_bytes = _lib.load().dyllm_fused_experts_workspace_bytes(T, top_k, E, hidden, inter)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("dyllm_fused_experts", _ptr(x), _ptr(ri), T, hidden, _ptr(w1), _ptr(w2), E, inter, _ptr(tw), _ptr(ti),
              top_k, _ptr(out), _ptr(orow), _ptr(ws), ws_bytes, _stream())
    return out
