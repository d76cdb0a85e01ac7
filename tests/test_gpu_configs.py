"""GPU parity at the full shapes of the benchmark configurations (LLaDA-8B config 1, Dream-7B
config 2 with GQA 28/4, LLaDA-MoE config 3, long-context config 4).

The HIP path runs on the whole batch; the oracle checks a seeded sample of rows. Every output
row of the sparse attention step depends only on its own query row and on its sequence's K, dV
and cached context, and every FFN/MoE output row only on its own input row, so the oracle run on
the sampled rows (with their sequences' keys) yields exactly the rows the full oracle would. The
index work (compaction of the full mask, the V-cache update) is checked on every row.
"""
import numpy as np
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close, assert_routing_weights, assert_mask_equal

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
D = 128

# name: (B, prompt, response, H, Hkv, salient fraction of the response rows)
ATTN_CASES = {
    "config1_llada8b": (8, 256, 768, 32, 32, 0.15),
    "config2_dream_p05": (16, 512, 1536, 28, 4, 0.05),
    "config2_dream_p50": (16, 512, 1536, 28, 4, 0.50),
    "config3_lladamoe": (32, 256, 768, 16, 16, 0.15),
    "config4_long": (2, 2048, 6144, 32, 32, 0.05),
}
N_SAMPLE = 48    # random rows across the batch, beside one whole sequence


def _rand(g, *shape, dev, std=1.0):
    x = torch.empty(*shape, dtype=torch.float32, device=dev)
    x.normal_(0.0, std, generator=g)
    return x.to(BF)


def _sub_batch(rows, cu_q, cu_k):
    """Sampled query rows grouped by sequence: (sequences, cu_q of the sample, cu_k and key-row
    index of those sequences)."""
    seqs = np.searchsorted(cu_q, rows, side="right") - 1
    uniq = np.unique(seqs)
    cu_qs = np.concatenate([[0], np.cumsum([(seqs == b).sum() for b in uniq])]).astype(np.int64)
    lens = [cu_k[b + 1] - cu_k[b] for b in uniq]
    cu_ks = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    krows = np.concatenate([np.arange(cu_k[b], cu_k[b + 1]) for b in uniq])
    return seqs, uniq, cu_qs, cu_ks, krows


@pytest.mark.parametrize("q_pruned", [True, False])
@pytest.mark.parametrize("case", list(ATTN_CASES))
def test_sparse_attention_step_full_shape(dev, case, q_pruned):
    from dyllm_amd.model_executor.layers.attention import Attention
    from dyllm_amd.utils.context import set_context
    from dyllm_amd.utils.metadata import get_metadata

    B, P, R, H, Hkv, frac = ATTN_CASES[case]
    print(f"[configs] attention {case} q_pruned={q_pruned}", flush=True)
    g = torch.Generator(device=dev).manual_seed(7)
    rng = np.random.default_rng(7)
    L = P + R
    Tk = B * L
    Tq = B * R if q_pruned else Tk
    cu_k = np.arange(B + 1, dtype=np.int64) * L
    cu_q = np.arange(B + 1, dtype=np.int64) * (R if q_pruned else L)
    cu_p = np.arange(B + 1, dtype=np.int64) * P
    i32 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int32, device=dev)
    i64 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int64, device=dev)
    md = get_metadata()
    md.running_seqs = list(range(B))
    md.running_seqs_tensor = torch.arange(B, device=dev)
    md.finished_seqs = []
    # full step: caches filled by the dense path
    set_context(True, cu_seqlens_q=i32(cu_k), cu_seqlens_q_cpu=cu_k.tolist(), cu_seqlens_k=i32(cu_k),
                cu_seqlens_k_cpu=cu_k.tolist(), max_seqlen_q=L, max_seqlen_k=L, context_lens_cpu=[L] * B,
                total_seqlen=Tk, total_seqlen_k=Tk)
    attn = Attention(H, D, D ** -0.5, Hkv, 0.99, device=dev)
    q_all, k_all, v_all = _rand(g, Tk, H, D, dev=dev), _rand(g, Tk, Hkv, D, dev=dev), _rand(g, Tk, Hkv, D, dev=dev)
    o_full = attn(q_all, k_all, v_all)
    # salient rows of this step: a fraction of every sequence's response rows
    n_per = max(1, int(round(frac * R)))
    sel = [np.sort(rng.choice(R, size=n_per, replace=False)) for _ in range(B)]
    idx_k = np.concatenate([cu_k[b] + P + sel[b] for b in range(B)])
    idx_q = np.concatenate([cu_q[b] + (0 if q_pruned else P) + sel[b] for b in range(B)])
    cu_s = np.arange(B + 1, dtype=np.int64) * n_per
    v_new = (v_all[i64(idx_k)].float() + 0.5 * _rand(g, len(idx_k), Hkv, D, dev=dev).float()).to(BF)
    k_new = k_all.clone()
    k_new[i64(idx_k)] = (k_all[i64(idx_k)].float() + 0.5 * _rand(g, len(idx_k), Hkv, D, dev=dev).float()).to(BF)
    resp = np.concatenate([np.arange(cu_k[b] + P, cu_k[b + 1]) for b in range(B)]) if q_pruned else np.arange(Tk)
    q = q_all[i64(resp)].contiguous()
    c_old = o_full[i64(resp)].cpu() if q_pruned else o_full.cpu()
    v_saved, c_saved = attn.v_cache.cache.clone(), attn.context_cache.cache.clone()
    # a stand-in FFN cache laid out differently from the attention caches: the step's compaction
    # also returns the rows of the next salient set in it
    from types import SimpleNamespace
    ffn_starts = torch.as_tensor(np.arange(B)[::-1].copy() * (L + 37) + 11, dtype=torch.int64, device=dev)
    attn.ffn_cache = SimpleNamespace(seq_start_gpu=ffn_starts)

    def run(tau):
        attn.threshold = tau
        attn.v_cache.cache.copy_(v_saved)
        attn.context_cache.cache.copy_(c_saved)
        ctx = set_context(False, cu_seqlens_q=i32(cu_q), cu_seqlens_q_cpu=cu_q.tolist(), cu_seqlens_k=i32(cu_k),
                          cu_seqlens_k_cpu=cu_k.tolist(), cu_promptlens=i32(cu_p), max_seqlen_q=int(cu_q[1]),
                          max_seqlen_k=L, context_lens_cpu=[L] * B, cu_salientlens=i32(cu_s),
                          idx_salient_row=i64(idx_q), idx_salient_row_k=i64(idx_k) if q_pruned else None,
                          max_salientlen=n_per, total_seqlen=Tq, total_seqlen_k=Tk)
        out = attn(q, k_new, v_new)
        return ctx, out

    # tau at the cosine quantile that makes about `frac` of the rows salient
    run(0.99)
    cos_gpu = ref.cosine_from_stats(attn._bufs.stats.cpu()).numpy()
    tau = float(np.quantile(cos_gpu, frac))
    ctx, out = run(tau)
    torch.cuda.synchronize()
    mask_gpu = attn._bufs.mask.cpu().numpy()
    stats_gpu = attn._bufs.stats.cpu()

    # compaction of the whole mask: bit-exact
    idx_ref, cu_ref = ref.compact(mask_gpu, cu_q)
    assert np.array_equal(ctx.idx_salient_row.cpu().numpy(), idx_ref)
    assert np.array_equal(ctx.cu_salientlens.cpu().numpy(), cu_ref)
    kspace = ref.fused_offset(idx_ref, cu_p, cu_ref) if q_pruned else idx_ref
    if q_pruned:
        assert np.array_equal(ctx.idx_salient_row_k.cpu().numpy(), kspace)
    seg = np.searchsorted(cu_k, kspace, side="right") - 1
    want_dest = ffn_starts.cpu().numpy()[seg] + (kspace - cu_k[seg])
    assert np.array_equal(attn._bufs.dest_rows[:len(idx_ref)].cpu().numpy(), want_dest)
    assert 0 < len(idx_ref) < Tq
    # V cache: the salient key rows hold the new V rows, every other row is unchanged
    v_after = attn.v_cache.cache.view(Tk, Hkv, D)
    want_v = v_saved.view(Tk, Hkv, D).clone()
    want_v[i64(idx_k)] = v_new
    assert torch.equal(v_after, want_v)

    # oracle on sampled rows: some salient input rows, the rest uniform
    sal_in = np.zeros(Tq, bool)
    sal_in[idx_q] = True
    pick = np.concatenate([rng.choice(idx_q, size=N_SAMPLE // 4, replace=False),
                           rng.choice(np.nonzero(~sal_in)[0], size=N_SAMPLE - N_SAMPLE // 4, replace=False)])
    # plus every row of the first sequence (up to 1024 rows): the whole salient set of a sequence
    # is then checked against the oracle, not a sample of it
    whole = np.arange(cu_q[0], min(cu_q[1], cu_q[0] + 1024))
    rows = np.union1d(pick, whole)
    seqs, uniq, cu_qs, cu_ks, krows = _sub_batch(rows, cu_q, cu_k)
    kr = i64(krows)
    k_sub = k_new[kr].cpu()
    v_cache_sub = want_v[kr].cpu()
    # dV over the sub-batch keys (bf16 tensor arithmetic, attention.py:70-73)
    vd_full = torch.zeros(Tk, Hkv, D, dtype=torch.float32)
    vd_full[torch.from_numpy(idx_k)] = ref.bf16_round(v_new.cpu().float() - v_saved.view(Tk, Hkv, D).cpu()[
        torch.from_numpy(idx_k)].float())
    vd_sub = vd_full[torch.from_numpy(krows)].to(BF)
    q_sub = q[i64(rows)].cpu()
    sal_pos = np.nonzero(sal_in[rows])[0]               # positions (within the sample) of salient rows
    cu_ss = np.concatenate([[0], np.cumsum([np.isin(np.nonzero(seqs == b)[0], sal_pos).sum() for b in uniq])])
    o_sal = ref.flash_attn_varlen(q_sub[torch.from_numpy(sal_pos)], k_sub, v_cache_sub, cu_ss, cu_ks)
    want_o, want_st, want_m = ref.attention_sparse_varlen(q_sub, k_sub, vd_sub, c_old[torch.from_numpy(rows)],
                                                          o_sal, cu_qs, cu_ks, sal_pos, tau)
    assert_bf16_close(out[i64(rows)], want_o, what=f"{case} new context")
    cos_ref = ref.cosine_from_stats(want_st).numpy()
    assert_mask_equal(mask_gpu[rows], want_m.numpy(), cos_ref, tau)
    assert torch.allclose(stats_gpu[torch.from_numpy(rows)], want_st, rtol=2e-3, atol=1e-2)
    # the context cache holds the new rows of every queried row
    cc = attn.context_cache.cache.view(Tk, H, D)
    assert torch.equal(cc[i64(resp)], out)


# name: (queried rows, hidden, inter, salient fraction)
FFN_CASES = {
    "config1_llada8b": (6144, 4096, 12288, 0.15),
    "config2_dream_p25": (24576, 3584, 18944, 0.25),
    "config4_long": (12288, 4096, 12288, 0.05),
}


@pytest.mark.parametrize("case", list(FFN_CASES))
def test_gathered_ffn_full_shape(dev, case):
    """Product FFN path at full shape: salient count read from device memory (no host sync),
    gather inside gate_up, split-K down GEMM scattering into cache rows."""
    from dyllm_amd import ops

    T, hid, inter, frac = FFN_CASES[case]
    print(f"[configs] ffn {case}", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    rng = np.random.default_rng(11)
    x = _rand(g, T, hid, dev=dev)
    wgu = _rand(g, 2 * inter, hid, dev=dev, std=hid ** -0.5)
    wd = _rand(g, hid, inter, dev=dev, std=inter ** -0.5)
    n = int(round(frac * T))
    rows = np.sort(rng.choice(T, size=n, replace=False))
    cap = torch.full((T,), -7, dtype=torch.int32, device=dev)     # capacity-sized, tail unused
    cap[:n] = torch.as_tensor(rows, dtype=torch.int32, device=dev)
    count = torch.tensor([n], dtype=torch.int32, device=dev)
    h = ops.ffn_gate_up(x, wgu, rows_idx=cap, count=count, hint=n)
    slab = torch.zeros(T + 64, hid, dtype=BF, device=dev)
    dest = torch.full((T,), -1, dtype=torch.int64, device=dev)
    dest[:n] = torch.as_tensor(rows, dtype=torch.int64, device=dev) + 64
    ops.ffn_down(h, wd, out=slab, out_rows=dest, count=count, hint=n)
    torch.cuda.synchronize()
    # exact-size path agrees with the device-count path
    y_exact = ops.swiglu_ffn(x, wgu, wd, rows_idx=torch.as_tensor(rows, dtype=torch.int32, device=dev))
    assert_bf16_close(slab[64:][torch.as_tensor(rows, device=dev)], y_exact, max_abs=1e-2, mean_rel=5e-4,
                      what="device-count vs exact-count FFN")
    untouched = torch.ones(T + 64, dtype=torch.bool, device=dev)
    untouched[dest[:n]] = False
    assert bool((slab[untouched] == 0).all())
    # oracle on sampled salient rows
    samp = np.sort(rng.choice(n, size=32, replace=False))
    xs = x[torch.as_tensor(rows[samp], device=dev)].cpu()
    want = ref.swiglu_ffn(xs, wgu.cpu(), wd.cpu()).to(BF)
    assert_bf16_close(y_exact[torch.as_tensor(samp, device=dev)], want, what=f"{case} SwiGLU")


def test_moe_full_shape_config3(dev):
    """LLaDA-MoE config 3: 15% of 32 x 768 response rows routed over 64 experts, top-8,
    hidden 2048, expert FFN 1024."""
    from dyllm_amd import ops

    print("[configs] moe config3", flush=True)
    T, hid, E, top_k, inter = 32 * 768, 2048, 64, 8, 1024
    g = torch.Generator(device=dev).manual_seed(5)
    rng = np.random.default_rng(5)
    n = int(round(0.15 * T))
    x = _rand(g, n, hid, dev=dev)
    wr = _rand(g, E, hid, dev=dev, std=hid ** -0.5)        # router logits ~ N(0, 1)
    # per-expert router bias ~ N(0, 0.5) for a skewed expert load, carried by a constant input
    # feature (the router has no bias term, fused_moe.py:375-408): x[:, 0] = 1, wr[:, 0] = bias
    x[:, 0] = 1.0
    wr[:, 0] = _rand(g, E, dev=dev, std=0.5)
    w1 = _rand(g, E, 2 * inter, hid, dev=dev, std=hid ** -0.5)
    w2 = _rand(g, E, hid, inter, dev=dev, std=inter ** -0.5)
    w, ids = ops.moe_gate(x, wr, top_k)
    out = ops.fused_experts(x, w1, w2, w, ids)
    torch.cuda.synchronize()
    load = torch.bincount(ids.reshape(-1).long().cpu(), minlength=E)
    assert load.max().item() > 3 * load.float().mean().item()   # the bias skews the expert load
    samp = torch.as_tensor(np.sort(rng.choice(n, size=32, replace=False)))
    xs = x.cpu()[samp]
    w_ref, ids_ref = ref.moe_gate(xs, wr.cpu(), top_k)
    # routing: identical expert sets wherever the oracle's k-th and (k+1)-th probabilities are
    # separated (a near-tie may legitimately resolve either way under a different sum order)
    probs = torch.softmax(xs.float() @ wr.cpu().float().t(), dim=-1)
    top = probs.topk(top_k + 1, dim=-1).values
    clear = (top[:, top_k - 1] - top[:, top_k]) > 1e-5
    got_ids = ids.cpu()[samp]
    assert torch.equal(got_ids[clear], ids_ref[clear])
    assert_routing_weights(w.cpu()[samp][clear], w_ref[clear])
    # experts, with the routing the device chose
    want = ref.naive_experts(xs, w1.cpu(), w2.cpu(), w.cpu()[samp], got_ids)
    assert_bf16_close(out.cpu()[samp], want.to(BF), what="MoE experts")
