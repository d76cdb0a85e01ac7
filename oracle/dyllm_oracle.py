"""CPU restatement of DyLLM's per-layer saliency hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker that the HIP path is compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it;
the product path (``dyllm_amd``) never does, and fails loudly when its HIP library is
missing instead of falling back here.

Everything runs on the CPU in fp32 torch (floating-point work) or numpy (integer /
index work). Each function cites the reference file:line whose semantics it restates
(paths relative to the DyLLM source tree). How each function is pinned:

* ``cosine_mask``               -- the reference's known-answer test
                                   (tests/test_parallelism.py:34-44), golden fixture.
* ``attention_sparse_varlen``   -- linearity invariant: with C_old = attn(Q,K,V_old) and
                                   dV = V_new - V_old, C_old + softmax(QK^T)dV == attn(Q,K,V_new);
                                   plus stats == closed-form dot/norms of the output.
* ``flash_attn_varlen``         -- torch.nn.functional.scaled_dot_product_attention per seq.
* ``compact`` / ``fused_offset``-- brute-force Python loops on small inputs, sortedness,
                                   per-seq count invariants.
* cache ops                     -- brute-force per-row Python loops.
* ``swiglu_ffn``                -- textbook F.silu(g) * u composition vs per-row loop.
* ``moe_gate`` / ``naive_experts`` -- per-token brute-force loop over the top-k experts.
* ``moe_align_block_size``      -- invariants (permutation, padding, expert ownership).
* ``rope_neox`` / ``rope_tables`` -- position 0 is the identity, each (d, d+64) pair keeps
                                   its length, and the result equals the complex product
                                   (x1 + i x2) e^{i p theta_d} (textbook RoPE).
* ``rms_norm`` / ``add_rms_norm`` -- unit RMS before the weight, weight applied per column;
                                   the fused form equals rms_norm of the fp32 sum (zero residual:
                                   identical to rms_norm) and a per-row loop.
* ``salient_kv_project``        -- composition of the above with a per-row loop linear.
* ``sparse_attention_step``     -- every queried row equals exact SDPA attn(Q, K, V_new) to bf16
                                   rounding, the V cache changes exactly at the salient K rows,
                                   the next set equals {cos(exact, C_old) < tau}, each K-space
                                   index is the same token as its Q-space index; composition
                                   mistakes (o_sal from the old V cache, dV at Q rows, a wrong
                                   prompt offset) are shown to fail; and the config-0 known
                                   answer (salient set == perturbed rows) through the whole step.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

BF16 = torch.bfloat16

# Key-block width of the reference's online softmax for head_dim 128
# (attn_tile_config.h:10-12 / DyllmTileDefault<128>::BLOCK_K = 64). The bf16 rounding
# of P happens relative to the running max of each such block.
ATTN_BLOCK_K = 64
# log2(e) as used by the reference's log2-domain softmax (attention_ops_kernels_sm80.cu:166-168).
LOG2E = 1.4426950408889634


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 -> bf16 (round-to-nearest-even) and back to fp32."""
    return x.to(BF16).float()


# ---------------------------------------------------------------------------
# (a7) tau test
# ---------------------------------------------------------------------------
def cosine_mask(stats: torch.Tensor, threshold: float) -> torch.Tensor:
    """Return ``cos < threshold`` from additive fp32 stats.

    Follows dyllm/distributed/parallel_state.py:62-66 (world size 1):
    ``cos = s0 * rsqrt(max(s1, 1e-8)) * rsqrt(max(s2, 1e-8))``.
    ``stats[:, 0]`` = dot, ``stats[:, 1]``/``[:, 2]`` = the two squared norms.
    """
    stats = stats.float()
    dot = stats[..., 0]
    n1 = stats[..., 1].clamp_min(1e-8)
    n2 = stats[..., 2].clamp_min(1e-8)
    cos = dot * torch.rsqrt(n1) * torch.rsqrt(n2)
    return cos < threshold


def cosine_from_stats(stats: torch.Tensor) -> torch.Tensor:
    """fp64 cosine of the same stats, used to find rows within the tau band."""
    s = stats.double()
    return s[:, 0] / torch.sqrt(s[:, 1].clamp_min(1e-8)) / torch.sqrt(s[:, 2].clamp_min(1e-8))


def saliency_stats(c_new: torch.Tensor, c_old: torch.Tensor) -> torch.Tensor:
    """Per-row ``{sum new*old, sum new^2, sum old^2}`` in fp32 (closed form of the
    reference's epilogue, attention_ops_kernels_sm80.cu:436-443 and
    attention_aux_kernels.cu:37-42). Accumulated in fp64 then rounded, so it is the
    order-independent value every fp32 summation order approximates."""
    n = c_new.double().reshape(c_new.shape[0], -1)
    o = c_old.double().reshape(c_old.shape[0], -1)
    return torch.stack([(n * o).sum(-1), (n * n).sum(-1), (o * o).sum(-1)], dim=-1).float()


# ---------------------------------------------------------------------------
# (a3)/(a15) textbook varlen attention (the flash_attn_varlen_func call sites)
# ---------------------------------------------------------------------------
def _online_softmax_pv(qb, kb, vb, c2, block_k):
    """Blocked log2-domain online softmax with P rounded to bf16 before P.V (the arithmetic
    of attention_ops_kernels_sm80.cu:282-381, which flash-attn 2 shares): per key block,
    m_new = max(m, rowmax), rescale = 2^((m - m_new) c2), p = 2^(s c2 - m_new c2),
    l = l*rescale + sum p (fp32), acc = acc*rescale + bf16(p) V. Returns (acc, l)."""
    H, Lq, D = qb.shape
    Lk = kb.shape[1]
    m = torch.full((H, Lq, 1), -3.4028234663852886e38)
    l = torch.zeros(H, Lq, 1)
    acc = torch.zeros(H, Lq, vb.shape[-1])
    for j0 in range(0, Lk, block_k):
        j1 = min(j0 + block_k, Lk)
        s = torch.matmul(qb, kb[:, j0:j1].transpose(1, 2))  # raw scores
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        rescale = torch.exp2((m - m_new) * c2)
        p = torch.exp2(s * c2 - m_new * c2)
        l = l * rescale + p.sum(-1, keepdim=True)
        acc = acc * rescale + torch.matmul(bf16_round(p), vb[:, j0:j1])
        m = m_new
    return acc, l


def flash_attn_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, scale=None, out_dtype=BF16, bf16_p=True):
    """Non-causal per-sequence softmax(QK^T*scale)V, as called at attention.py:41-52
    and :76-87 (flash-attn 2.8.3, not vendored). q:[Tq,H,D], k/v:[Tk,Hkv,D] (GQA: query
    head h uses kv head h // (H/Hkv)). fp32 math; with ``bf16_p`` the probabilities are
    rounded to bf16 before the PV product inside 64-key online-softmax blocks, as
    flash-attn does for bf16 inputs; output rounded to ``out_dtype``."""
    Tq, H, D = q.shape
    Hkv = k.shape[1]
    g = H // Hkv
    scale = D ** -0.5 if scale is None else scale
    c2 = float(np.float32(np.float32(scale) * np.float32(LOG2E)))
    out = torch.zeros(Tq, H, D, dtype=torch.float32)
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        if qe == qs or ke == ks:
            continue
        qb = q[qs:qe].float().transpose(0, 1)  # H, Lq, D
        kb = k[ks:ke].float().transpose(0, 1).repeat_interleave(g, dim=0)
        vb = v[ks:ke].float().transpose(0, 1).repeat_interleave(g, dim=0)
        if bf16_p:
            acc, l = _online_softmax_pv(qb, kb, vb, c2, ATTN_BLOCK_K)
            o = acc / l
        else:
            s = torch.matmul(qb, kb.transpose(1, 2)) * scale
            o = torch.matmul(torch.softmax(s, dim=-1), vb)
        out[qs:qe] = o.transpose(0, 1)
    return out.to(out_dtype) if out_dtype is not None else out


# ---------------------------------------------------------------------------
# (a4) K block masks
# ---------------------------------------------------------------------------
def k_block_masks(idx_salient_k, cu_salientlens, cu_seqlens_k, max_seqlen_k, block_k=ATTN_BLOCK_K):
    """uint64 bitmask per (seq, key block) of salient key rows
    (attention_aux_kernels.cu:74-110). Returns numpy uint64 [B, cdiv(max_k, block_k)]."""
    cu_k = np.asarray(cu_seqlens_k, dtype=np.int64)
    cu_s = np.asarray(cu_salientlens, dtype=np.int64)
    idx = np.asarray(idx_salient_k, dtype=np.int64)
    B = len(cu_k) - 1
    nblk = -(-int(max_seqlen_k) // block_k)
    out = np.zeros((B, nblk), dtype=np.uint64)
    for b in range(B):
        for r in idx[cu_s[b]:cu_s[b + 1]]:
            off = int(r - cu_k[b])
            if 0 <= off < cu_k[b + 1] - cu_k[b]:
                out[b, off // block_k] |= np.uint64(1) << np.uint64(off % block_k)
    return out


# ---------------------------------------------------------------------------
# (a5)+(a6)+(a7) column-sparse attention with saliency stats
# ---------------------------------------------------------------------------
def attention_sparse_varlen(Q, K, Vd, C, o_sal, cu_seqlens_q, cu_seqlens_k, idx_salient_row,
                            threshold, block_k=ATTN_BLOCK_K):
    """Restates ``attention_sparse_varlen`` (attention.cpp:64-179) for one layer.

    For every query row: ``new = C + softmax(Q K^T / sqrt(D)) dV`` with the reference's
    log2-domain online softmax over ``block_k``-wide key blocks, P rounded to bf16 before
    the P.dV product and the row sum kept in fp32 (attention_ops_kernels_sm80.cu:166-449).
    Non-salient rows: stats from the unrounded fp32 ``new`` (sm80.cu:436-443).
    Salient rows (``idx_salient_row``, Q space): output and stats from bf16 ``o_sal``
    (attention_aux_kernels.cu:22-72). Then the tau test (aux:10-20 / parallel_state.py:62-66).

    Q:[Tq,H,D] K,Vd:[Tk,Hkv,D] C:[Tq,H,D] o_sal:[n_sal,H,D] (bf16 values).
    Returns (O bf16 [Tq,H,D], stats fp32 [Tq,3], mask bool [Tq]).
    """
    Tq, H, D = Q.shape
    Hkv = K.shape[1]
    g = H // Hkv
    c2 = np.float32(1.0 / math.sqrt(D)) * np.float32(LOG2E)  # softmax_scale_log2 (fp32)
    c2 = float(np.float32(c2))
    newc = torch.zeros(Tq, H, D, dtype=torch.float32)
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        if qe == qs:
            continue
        qb = Q[qs:qe].float().transpose(0, 1)  # H,Lq,D
        kb = K[ks:ke].float().transpose(0, 1).repeat_interleave(g, dim=0)
        vb = Vd[ks:ke].float().transpose(0, 1).repeat_interleave(g, dim=0)
        acc, l = _online_softmax_pv(qb, kb, vb, c2, block_k)
        inv = 1.0 / l
        newc[qs:qe] = (C[qs:qe].float().transpose(0, 1) + acc * inv).transpose(0, 1)
    stats = saliency_stats(newc, C.float())
    out = newc.to(BF16)
    idx = torch.as_tensor(idx_salient_row, dtype=torch.long)
    if idx.numel():
        out[idx] = o_sal.to(BF16)
        stats[idx] = saliency_stats(o_sal.float(), C[idx].float())
    mask = cosine_mask(stats, threshold)
    return out, stats, mask


# ---------------------------------------------------------------------------
# (a8) compaction
# ---------------------------------------------------------------------------
def compact(mask, cu_seqlens_q):
    """``idxs = nonzero(mask)`` (ascending) and ``cu_salientlens = searchsorted(idxs,
    cu_seqlens_q)`` as at attention.py:147-150. Returns numpy (int64 [n], int32 [B+1])."""
    m = np.asarray(mask).astype(bool)
    idxs = np.nonzero(m)[0].astype(np.int64)
    cu = np.searchsorted(idxs, np.asarray(cu_seqlens_q, dtype=np.int64), side="left").astype(np.int32)
    return idxs, cu


def fused_offset(idxs, cu_promptlens, cu_salientlens):
    """K-space rows of Q-pruned salient indices, attention_aux_kernels.cu:112-128:
    ``out[t] = idxs[t] + cu_promptlens[seg(t)+1]`` where seg(t) is the sequence whose
    ``cu_salientlens`` range contains t."""
    idxs = np.asarray(idxs, dtype=np.int64)
    cp = np.asarray(cu_promptlens, dtype=np.int64)
    cs = np.asarray(cu_salientlens, dtype=np.int64)
    seg = np.searchsorted(cs[1:], np.arange(len(idxs)), side="right")
    return idxs + cp[seg + 1]


# ---------------------------------------------------------------------------
# (a9)/(a10)/(a14) cache ops over the packed row cache
# ---------------------------------------------------------------------------
def get_seqs(cache, seq_starts, cu, seq_ids, total_rows):
    """cache_kernels.cu:18-64: out[cu[b]+i] = cache[seq_starts[seq_ids[b]] + i]."""
    out = torch.zeros(total_rows, cache.shape[1], dtype=cache.dtype)
    for b in range(len(seq_ids)):
        s0 = int(seq_starts[int(seq_ids[b])])
        for i in range(int(cu[b + 1]) - int(cu[b])):
            out[int(cu[b]) + i] = cache[s0 + i]
    return out


def get_block(cache, seq_starts, cu_k, cu_q, seq_ids, total_rows):
    """cache_kernels.cu:200-247: the tail ``Lq`` rows of each cached sequence."""
    out = torch.zeros(total_rows, cache.shape[1], dtype=cache.dtype)
    for b in range(len(seq_ids)):
        L = int(cu_q[b + 1]) - int(cu_q[b])
        s0 = int(seq_starts[int(seq_ids[b])]) + int(cu_k[b + 1]) - int(cu_k[b]) - L
        for i in range(L):
            out[int(cu_q[b]) + i] = cache[s0 + i]
    return out


def reset_full(cache, x, seq_starts, cu, seq_ids):
    """cache_kernels.cu:110-156: cache[seq_starts[seq_ids[b]] + i] = x[cu[b]+i]."""
    cache = cache.clone()
    for b in range(len(seq_ids)):
        s0 = int(seq_starts[int(seq_ids[b])])
        for i in range(int(cu[b + 1]) - int(cu[b])):
            cache[s0 + i] = x[int(cu[b]) + i]
    return cache


def reset_block(cache, x, seq_starts, cu_k, cu_q, seq_ids):
    """cache_kernels.cu:296-343: write the tail ``Lq`` rows of each cached sequence."""
    cache = cache.clone()
    for b in range(len(seq_ids)):
        L = int(cu_q[b + 1]) - int(cu_q[b])
        s0 = int(seq_starts[int(seq_ids[b])]) + int(cu_k[b + 1]) - int(cu_k[b]) - L
        for i in range(L):
            cache[s0 + i] = x[int(cu_q[b]) + i]
    return cache


def scatter_update(cache, new_vals, row_idx, cu_seqlens, seq_starts, seq_ids):
    """cache_kernels.cu:388-426: row r (packed space) of sequence b goes to
    cache[seq_starts[seq_ids[b]] + r - cu[b]]."""
    cache = cache.clone()
    cu = [int(x) for x in cu_seqlens]
    for m, r in enumerate(row_idx):
        r = int(r)
        b = max(i for i in range(len(cu) - 1) if cu[i] <= r)
        cache[int(seq_starts[int(seq_ids[b])]) + r - cu[b]] = new_vals[m]
    return cache


def gather_rows_2D(x, idx):
    """utils/util.py:19-36 (torch.gather of whole rows)."""
    return x[torch.as_tensor(idx, dtype=torch.long)]


# ---------------------------------------------------------------------------
# (a12) SwiGLU FFN
# ---------------------------------------------------------------------------
def swiglu_ffn(x, w_gate_up, w_down):
    """LLaDAMLP.forward (llada.py:38-43) on the gathered rows: gate_up GEMM
    (linear.py:76-93), SiluAndMul (activations.py:11-14: ``silu(x[:, :I]) * x[:, I:]``),
    down GEMM (linear.py:216-220). fp32 math; the reference rounds the gate_up product to
    bf16, which is emulated so the comparison tolerance only has to absorb sum order."""
    gu = bf16_round(x.float() @ w_gate_up.float().t())
    I = gu.shape[1] // 2
    h = bf16_round(F.silu(gu[:, :I]) * gu[:, I:])
    return h @ w_down.float().t()


# ---------------------------------------------------------------------------
# (next) salient-row K/V projection: linear + k_norm + RoPE + K-cache scatter
# ---------------------------------------------------------------------------
def rope_tables(head_dim, max_position, base):
    """cos / sin tables of RotaryEmbedding.__init__ (rotary_embedding.py:19-38): fp32
    inv_freq = base^(-2i/D), freqs = positions x inv_freq; [max_position, D/2] each."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    f = torch.outer(torch.arange(max_position, dtype=torch.float32), inv)
    return f.cos(), f.sin()


def rope_neox(x, cos, sin, positions, max_position=None):
    """apply_rotary_emb (rotary_embedding.py:8-16) at clamped positions (:47-52): halves
    x1 | x2 of each head, y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin in fp32 (each product
    and sum rounded, no contraction), result rounded to bf16. x: [n, H, D] bf16."""
    mp = cos.shape[0] if max_position is None else max_position
    pos = torch.as_tensor(positions, dtype=torch.long).clamp(0, mp - 1)
    c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
    x1, x2 = x.float().chunk(2, dim=-1)
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(BF16)


def rms_norm(x, weight, eps):
    """RMSNorm.rms_forward (layernorm.py:15-24): fp32 mean of squares over the last dim,
    x * rsqrt(var + eps) rounded to bf16, then times the bf16 weight (rounded again)."""
    xf = x.float()
    y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(BF16)
    return (y.float() * weight.float()).to(BF16)


def add_rms_norm(x, residual, weight, eps):
    """RMSNorm.add_rms_forward (layernorm.py:29-37): s = x + residual in fp32, residual_out =
    bf16(s), y = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight). Returns (y, residual_out)."""
    sf = x.float() + residual.float()
    y = (sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + eps)).to(BF16)
    return (y.float() * weight.float()).to(BF16), sf.to(BF16)


def salient_kv_project(hidden, idx, w_kv, bias, positions, cos, sin, num_kv_heads, k_norm_weight=None, eps=1e-6):
    """The salient-row K/V path of the sparse step (llada.py:108-143, lladamoe.py:204-239):
    kv = kv_proj(hidden[idx]) (bf16 output of an fp32-accumulated product, plus bias),
    k -> optional per-head k_norm -> RoPE at positions[idx]; returns (k, v) bf16
    [n, Hkv, 128] -- k is what scatter_update writes into the K cache."""
    idx = torch.as_tensor(idx, dtype=torch.long)
    kv = hidden[idx].float() @ w_kv.float().t()
    if bias is not None:
        kv = kv + bias.float()
    kv = kv.to(BF16)
    kvs = w_kv.shape[0] // 2
    k = kv[:, :kvs].reshape(-1, num_kv_heads, 128)
    v = kv[:, kvs:].reshape(-1, num_kv_heads, 128)
    if k_norm_weight is not None:
        k = rms_norm(k, k_norm_weight, eps)
    return rope_neox(k, cos, sin, positions[idx]), v


# ---------------------------------------------------------------------------
# (a13) MoE
# ---------------------------------------------------------------------------
def moe_gate(x, router_weight, top_k, renormalize=False):
    """fused_moe.py:375-408 without the DiffusionGemma extras: fp32 router logits,
    softmax, top-k (torch.topk order), optional renormalisation; weights returned in
    x's dtype, ids int32."""
    logits = x.float() @ router_weight.float().t()
    probs = torch.softmax(logits, dim=-1)
    w, ids = torch.topk(probs, top_k, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.to(x.dtype), ids.to(torch.int32)


def naive_experts(x, w1, w2, topk_weights, topk_ids):
    """fused_moe.py:341-369 with activation='silu' (lladamoe.py:100): per expert,
    ``silu(g)*u`` of ``x @ w1[e]^T`` then ``@ w2[e]^T`` times the routing weight, summed
    over the top-k. fp32 math with the reference's bf16 rounding of the GEMM-1 output
    and of the gated activation (fused_moe.py:313-316)."""
    T, Hd = x.shape
    out = torch.zeros(T, Hd, dtype=torch.float32)
    for e in range(w1.shape[0]):
        tok, slot = (topk_ids == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        gu = bf16_round(x[tok].float() @ w1[e].float().t())
        I = gu.shape[1] // 2
        h = bf16_round(F.silu(gu[:, :I]) * gu[:, I:])
        y = bf16_round((h @ w2[e].float().t()) * topk_weights[tok, slot].float().unsqueeze(-1))
        out.index_add_(0, tok, y)
    return out


def moe_align_block_size(topk_ids, block_size, num_experts):
    """fused_moe.py:37-85: stable sort of flattened (token, k) slots by expert, each
    expert bucket padded to ``block_size`` with the sentinel ``T*top_k``.
    Returns numpy (sorted_token_ids int32, expert_ids int32, num_post_pad int)."""
    flat = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    total = flat.size
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts)
    padded = (counts + block_size - 1) // block_size * block_size
    out = []
    eids = []
    pos = 0
    for e in range(num_experts):
        mem = order[pos:pos + counts[e]]
        pos += counts[e]
        bucket = np.full(padded[e], total, dtype=np.int32)
        bucket[:counts[e]] = mem
        out.append(bucket)
        eids += [e] * (padded[e] // block_size)
    sorted_ids = np.concatenate(out) if out else np.zeros(0, np.int32)
    return sorted_ids.astype(np.int32), np.asarray(eids, dtype=np.int32), int(padded.sum())


# ---------------------------------------------------------------------------
# (a1) one sparse attention step, end to end (attention.py:64-178)
# ---------------------------------------------------------------------------
def sparse_attention_step(q, k_full, v_new, v_cache_packed, c_old, cu_seqlens_q, cu_seqlens_k,
                          cu_salientlens, idx_salient_row, idx_salient_row_k, cu_promptlens,
                          threshold):
    """The sparse branch of ``Attention.forward`` (attention.py:64-178) on packed tensors.

    v_cache_packed: [Tk,Hkv,D] cached V rows (``v_cache.get_seqs``); c_old: [Tq,H,D] the
    cached context rows for the queried rows (``get_seqs_block`` when Q-pruned).
    idx_salient_row_k is None in refresh mode. Returns a dict with the new context,
    the updated packed V, the stats/mask and the next salient index lists.
    """
    q_pruned = idx_salient_row_k is not None
    kidx = torch.as_tensor(idx_salient_row_k if q_pruned else idx_salient_row, dtype=torch.long)
    sidx = torch.as_tensor(idx_salient_row, dtype=torch.long)
    v_cache = v_cache_packed.clone()
    v_delta = v_new.float() - v_cache[kidx].float()                  # attention.py:70/73
    v_delta = bf16_round(v_delta)                                     # bf16 tensor arithmetic
    v_cache[kidx] = v_new.to(v_cache.dtype)                           # attention.py:71/74
    o_sal = flash_attn_varlen(q[sidx], k_full, v_cache, cu_salientlens, cu_seqlens_k)  # :76-87
    vd = torch.zeros_like(k_full, dtype=torch.float32)
    vd[kidx] = v_delta                                                # :89-96
    newc, stats, mask = attention_sparse_varlen(q, k_full, vd.to(BF16), c_old, o_sal,
                                                cu_seqlens_q, cu_seqlens_k, sidx, threshold)
    idxs, cu_sal = compact(mask.numpy(), cu_seqlens_q)               # :147-150
    idx_k = fused_offset(idxs, cu_promptlens, cu_sal) if q_pruned else None  # :152-166
    return dict(new_c=newc, v_cache=v_cache, o_sal=o_sal, stats=stats, mask=mask,
                idx_salient_row=idxs, cu_salientlens=cu_sal, idx_salient_row_k=idx_k)
