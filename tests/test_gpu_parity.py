"""GPU parity: every HIP entry point against the CPU oracle on seeded inputs.

Integer / index / copy work is compared bit-exactly; bf16 outputs within max abs 2e-2 and
mean relative 1e-3; salient sets bit-exactly outside a 1e-6 band around tau.
"""
import numpy as np
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close, assert_routing_weights, assert_mask_equal

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _ops():
    from dyllm_amd import ops

    return ops


def _gen(seed):
    g = torch.Generator().manual_seed(seed)
    return g


def _randn(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(BF)


# ---------------------------------------------------------------------------------------
# packed row caches
# ---------------------------------------------------------------------------------------
def _cache_case(seed=0, D=4096):
    g = _gen(seed)
    lens_k = [37, 128, 5]
    lens_q = [20, 128, 5]
    seq_ids = [7, 2, 4]
    starts = torch.full((16,), -1, dtype=torch.long)
    pos = 3
    for sid, L in zip(seq_ids, lens_k):
        starts[sid] = pos
        pos += L + 11
    cache = _randn(g, pos + 5, D)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32)
    return g, cache, starts, torch.tensor(seq_ids, dtype=torch.long), cu_k, cu_q


@pytest.mark.parametrize("D", [4096, 1024, 8])
def test_cache_ops_exact(dev, D):
    ops = _ops()
    g, cache, starts, sids, cu_k, cu_q = _cache_case(1, D)
    Tk, Tq = int(cu_k[-1]), int(cu_q[-1])
    c_d, st_d, id_d, cuk_d, cuq_d = (t.to(dev) for t in (cache, starts, sids, cu_k, cu_q))
    got = ops.get_seqs_cuda(c_d, st_d, cuk_d, id_d, Tk).cpu()
    assert torch.equal(got, ref.get_seqs(cache, starts, cu_k, sids, Tk))
    got = ops.get_block_cuda(c_d, st_d, cuk_d, cuq_d, id_d, Tq).cpu()
    assert torch.equal(got, ref.get_block(cache, starts, cu_k, cu_q, sids, Tq))
    xin = _randn(g, Tk, D)
    c2 = c_d.clone()
    ops.reset_full_cuda(c2, xin.to(dev), st_d, cuk_d, id_d, Tk)
    assert torch.equal(c2.cpu(), ref.reset_full(cache, xin, starts, cu_k, sids))
    xq = _randn(g, Tq, D)
    c3 = c_d.clone()
    ops.reset_block_cuda(c3, xq.to(dev), st_d, cuk_d, cuq_d, id_d, Tq)
    assert torch.equal(c3.cpu(), ref.reset_block(cache, xq, starts, cu_k, cu_q, sids))
    rows = torch.tensor([0, 36, 37, 100, 164, 169], dtype=torch.long)
    nv = _randn(g, rows.numel(), D)
    c4 = c_d.clone()
    ops.scatter_update_cuda(c4, nv.to(dev), rows.to(dev), cuk_d, st_d, id_d)
    assert torch.equal(c4.cpu(), ref.scatter_update(cache, nv, rows, cu_k, starts, sids))
    dest = ops.scatter_dest_rows(rows.to(dev), cuk_d, st_d, id_d).cpu()
    want = [int(starts[int(sids[int(np.searchsorted(cu_k.numpy(), int(r), 'right') - 1)])]) + int(r) -
            int(cu_k[int(np.searchsorted(cu_k.numpy(), int(r), 'right') - 1)]) for r in rows]
    assert dest.tolist() == want
    gi = torch.tensor([5, 5, 0, 169], dtype=torch.long)
    got = ops.gather_rows_2D(c_d, gi.to(dev)).cpu()
    assert torch.equal(got, ref.gather_rows_2D(cache, gi))
    # indices outside [0, rows) give zero rows; the kernel never reads outside x
    bad = torch.tensor([3, -1, cache.shape[0], 2], dtype=torch.long)
    got = ops.gather_rows_2D(c_d, bad.to(dev)).cpu()
    assert torch.equal(got[[0, 3]], cache[[3, 2]]) and not got[[1, 2]].any()


def test_cache_ops_many_sequences(dev):
    """Row lookups over more than 64 sequences (the ballot search takes the prefix array in 64-entry
    chunks), with empty sequences (equal prefix entries): every map bit-exact against the oracle."""
    ops = _ops()
    g = _gen(11)
    rng = np.random.default_rng(11)
    B, D = 150, 256
    lens_k = rng.integers(0, 9, size=B)
    lens_k[[0, 70, 149]] = 0
    lens_q = np.minimum(lens_k, rng.integers(0, 5, size=B))
    seq_ids = rng.permutation(200)[:B]
    starts = torch.full((200,), -1, dtype=torch.long)
    pos = 1
    for sid, L in zip(seq_ids, lens_k):
        starts[int(sid)] = pos
        pos += int(L) + 2
    cache = _randn(g, pos + 3, D)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32)
    sids = torch.tensor(seq_ids, dtype=torch.long)
    Tk, Tq = int(cu_k[-1]), int(cu_q[-1])
    c_d, st_d, id_d, cuk_d, cuq_d = (t.to(dev) for t in (cache, starts, sids, cu_k, cu_q))
    assert torch.equal(ops.get_seqs_cuda(c_d, st_d, cuk_d, id_d, Tk).cpu(), ref.get_seqs(cache, starts, cu_k, sids, Tk))
    assert torch.equal(ops.get_block_cuda(c_d, st_d, cuk_d, cuq_d, id_d, Tq).cpu(),
                       ref.get_block(cache, starts, cu_k, cu_q, sids, Tq))
    xin = _randn(g, Tk, D)
    c2 = c_d.clone()
    ops.reset_full_cuda(c2, xin.to(dev), st_d, cuk_d, id_d, Tk)
    assert torch.equal(c2.cpu(), ref.reset_full(cache, xin, starts, cu_k, sids))
    rows = torch.from_numpy(np.sort(rng.choice(Tk, size=min(Tk, 97), replace=False))).long()
    nv = _randn(g, rows.numel(), D)
    c4 = c_d.clone()
    ops.scatter_update_cuda(c4, nv.to(dev), rows.to(dev), cuk_d, st_d, id_d)
    assert torch.equal(c4.cpu(), ref.scatter_update(cache, nv, rows, cu_k, starts, sids))


# ---------------------------------------------------------------------------------------
# saliency, tau test, compaction
# ---------------------------------------------------------------------------------------
def test_saliency_stats_and_mask(dev):
    ops = _ops()
    g = _gen(2)
    T, D = 3001, 4096
    old = torch.randn(T, D, generator=g)
    new = old.clone()
    pert = torch.rand(T, generator=g) < 0.3
    new[pert] += 0.1 * torch.randn(int(pert.sum()), D, generator=g) * torch.rand(int(pert.sum()), 1, generator=g)
    old, new = old.to(BF), new.to(BF)
    want_stats = ref.saliency_stats(new.float(), old.float())
    cos = ref.cosine_from_stats(want_stats).numpy()
    tau = float(np.median(cos[pert.numpy()]))
    stats, mask = ops.saliency_stats(new.to(dev), old.to(dev), tau)
    torch.testing.assert_close(stats.cpu(), want_stats, rtol=2e-6, atol=1e-3)
    assert_mask_equal(mask.cpu().numpy(), cos < tau, cos, tau)
    # tau test from the stats alone (parallel_state.py:62-66)
    m2 = ops.tensor_parallel_cosine_mask(want_stats.to(dev), tau).cpu()
    assert_mask_equal(m2.numpy(), ref.cosine_mask(want_stats, tau).numpy(), cos, tau, band=2e-7)


@pytest.mark.parametrize("T,density,B", [(0, 0.0, 1), (1, 1.0, 1), (6144, 0.15, 8), (40000, 0.5, 16),
                                         (16385, 0.01, 3), (4096, 1.0, 2)])
def test_compaction_exact(dev, T, density, B):
    ops = _ops()
    rng = np.random.default_rng(T + B)
    mask = rng.random(T) < density
    cuts = np.sort(rng.integers(0, T + 1, size=B - 1)) if B > 1 else np.zeros(0, np.int64)
    cu_q = np.concatenate([[0], cuts, [T]]).astype(np.int32)
    cu_p = np.concatenate([[0], np.cumsum(rng.integers(0, 300, size=B))]).astype(np.int32)
    res = ops.salient_compact(torch.from_numpy(mask).to(dev), torch.from_numpy(cu_q).to(dev),
                              torch.from_numpy(cu_p).to(dev))
    idx64, idx32, idxk, cu_sal = res.trimmed()
    want_idx, want_cu = ref.compact(mask, cu_q)
    assert res.n() == want_idx.size
    assert np.array_equal(idx64.cpu().numpy(), want_idx)
    assert np.array_equal(idx32.cpu().numpy(), want_idx.astype(np.int32))
    assert np.array_equal(cu_sal.cpu().numpy(), want_cu)
    assert np.array_equal(idxk.cpu().numpy(), ref.fused_offset(want_idx, cu_p, want_cu))


def test_fused_offset_launch(dev):
    ops = _ops()
    rng = np.random.default_rng(5)
    B = 5
    counts = rng.integers(0, 40, size=B)
    cu_sal = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    cu_p = np.concatenate([[0], np.cumsum(rng.integers(1, 64, size=B))]).astype(np.int32)
    n = int(cu_sal[-1])
    idxs = rng.integers(0, 1000, size=n).astype(np.int32)
    out = torch.full((n + 7,), -5, dtype=torch.int64, device=dev)
    ops.fused_offset_launch(torch.from_numpy(idxs).to(dev), torch.tensor([n], dtype=torch.int32, device=dev),
                            torch.from_numpy(cu_p).to(dev), torch.from_numpy(cu_sal).to(dev), out, n + 7)
    got = out.cpu().numpy()
    assert np.array_equal(got[:n], ref.fused_offset(idxs, cu_p, cu_sal))
    assert (got[n:] == -5).all()


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------
def _attn_lens():
    return [(70, 200), (128, 128), (1, 65), (200, 300)]  # (Lq, Lk)


@pytest.mark.parametrize("H,Hkv", [(4, 4), (4, 2), (7, 1)])
def test_flash_attn_dense_and_rowsparse(dev, H, Hkv):
    ops = _ops()
    g = _gen(3 + H)
    lens = _attn_lens()
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum([a for a, _ in lens])]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum([b for _, b in lens])]), dtype=torch.int32)
    Tq, Tk = int(cu_q[-1]), int(cu_k[-1])
    q, k, v = _randn(g, Tq, H, 128), _randn(g, Tk, Hkv, 128), _randn(g, Tk, Hkv, 128)
    o = ops.flash_attn_varlen_func(q.to(dev), k.to(dev), v.to(dev), cu_q.to(dev), cu_k.to(dev), 200, 300)
    want = ref.flash_attn_varlen(q, k, v, cu_q, cu_k)
    assert_bf16_close(o, want, what="dense attention")
    # row-sparse: a sorted subset of rows per sequence
    rng = np.random.default_rng(H)
    rows, cu_s = [], [0]
    for b in range(len(lens)):
        sel = np.sort(rng.choice(np.arange(int(cu_q[b]), int(cu_q[b + 1])), size=max(1, lens[b][0] // 3), replace=False))
        rows += sel.tolist()
        cu_s.append(len(rows))
    rows_t = torch.tensor(rows, dtype=torch.int32)
    cu_s_t = torch.tensor(cu_s, dtype=torch.int32)
    o2 = ops.flash_attn_varlen_func(q.to(dev), k.to(dev), v.to(dev), cu_s_t.to(dev), cu_k.to(dev), 200, 300,
                                    q_rows=rows_t.to(dev))
    want2 = ref.flash_attn_varlen(q[rows_t.long()], k, v, cu_s_t, cu_k)
    assert_bf16_close(o2, want2, what="row-sparse attention")


def _colsparse_case(seed, H, Hkv, q_pruned, lens=None, sal_frac=0.15):
    """Inputs shaped like one sparse step (attention.py:64-139)."""
    g = _gen(seed)
    rng = np.random.default_rng(seed)
    lens = lens or [(96, 160), (200, 256), (33, 97)]   # (prompt, response) per sequence
    Lk = [p + r for p, r in lens]
    Lq = [r if q_pruned else p + r for p, r in lens]
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_p = np.concatenate([[0], np.cumsum([p for p, _ in lens])]).astype(np.int32)
    Tq, Tk = int(cu_q[-1]), int(cu_k[-1])
    D = 128
    q = _randn(g, Tq, H, D)
    k = _randn(g, Tk, Hkv, D)
    v_old = _randn(g, Tk, Hkv, D)
    c_old = ref.flash_attn_varlen(q, k, v_old, cu_q, cu_k)
    # salient rows: response rows only, per sequence ascending
    idx_q, idx_k, cu_s = [], [], [0]
    for b, (p, r) in enumerate(lens):
        sel = np.sort(rng.choice(r, size=max(1, int(r * sal_frac)), replace=False))
        idx_k += (cu_k[b] + p + sel).tolist()
        idx_q += ((cu_q[b] + sel) if q_pruned else (cu_q[b] + p + sel)).tolist()
        cu_s.append(len(idx_q))
    idx_q = np.asarray(idx_q, np.int32)
    idx_k = np.asarray(idx_k, np.int32)
    v_new_rows = (v_old[idx_k].float() + 0.7 * torch.randn(len(idx_k), Hkv, D, generator=g)).to(BF)
    v_cache = v_old.clone()
    v_cache[idx_k] = v_new_rows
    dv = torch.zeros(Tk, Hkv, D, dtype=BF)
    dv[idx_k] = (v_new_rows.float() - v_old[idx_k].float()).to(BF)
    o_sal = ref.flash_attn_varlen(q[torch.from_numpy(idx_q).long()], k, v_cache, cu_s, cu_k)
    return dict(q=q, k=k, dv=dv, c=c_old, o_sal=o_sal, cu_q=cu_q, cu_k=cu_k, cu_s=np.asarray(cu_s, np.int32),
                cu_p=cu_p, idx_q=idx_q, idx_k=idx_k, maxq=max(Lq), maxk=max(Lk))


@pytest.mark.parametrize("q_pruned", [True, False])
@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2)])
def test_attention_sparse_varlen(dev, q_pruned, H, Hkv):
    ops = _ops()
    cs = _colsparse_case(11 + H + int(q_pruned), H, Hkv, q_pruned)
    Tq = cs["q"].shape[0]
    # oracle at tau = 0.99 first to pick a tau in the middle of the cosine distribution
    _, st0, _ = ref.attention_sparse_varlen(cs["q"], cs["k"], cs["dv"], cs["c"], cs["o_sal"], cs["cu_q"],
                                            cs["cu_k"], cs["idx_q"], 0.99)
    cos = ref.cosine_from_stats(st0).numpy()
    tau = float(np.median(cos))
    want_o, want_st, want_m = ref.attention_sparse_varlen(cs["q"], cs["k"], cs["dv"], cs["c"], cs["o_sal"],
                                                          cs["cu_q"], cs["cu_k"], cs["idx_q"], tau)
    t = lambda a: torch.as_tensor(a).to(dev)
    stats = torch.zeros(Tq, 3, dtype=torch.float32, device=dev)
    mask = torch.empty(Tq, dtype=torch.bool, device=dev)
    o = ops.attention_sparse_varlen(t(cs["q"]), t(cs["k"]), t(cs["dv"]), t(cs["c"]), t(cs["o_sal"]), t(cs["cu_q"]),
                                    t(cs["cu_k"]), cs["maxq"], cs["maxk"], Tq, t(cs["cu_s"]), t(cs["idx_q"]), stats,
                                    mask, tau, q_pruned, t(cs["idx_k"]) if q_pruned else None)
    assert_bf16_close(o, want_o, what="column-sparse output")
    # salient rows are copied bit-exactly from o_sal
    assert torch.equal(o.cpu()[torch.from_numpy(cs["idx_q"]).long()], cs["o_sal"])
    torch.testing.assert_close(stats.cpu(), want_st, rtol=1e-4, atol=1e-2)
    excluded = assert_mask_equal(mask.cpu().numpy(), want_m.numpy(), cos, tau)
    assert excluded < Tq // 20


@pytest.mark.parametrize("lens,sal_frac,H,Hkv", [
    # most keys salient: up to 4 sixteen-key groups per 64-key block, ragged last blocks
    ([(30, 290), (100, 157), (5, 60)], 0.6, 4, 2),
    # 4096 keys (the largest two-pass sequence) next to 4200 (the single-pass path) in one launch
    ([(64, 4032), (200, 4000)], 0.05, 2, 1),
])
def test_attention_sparse_varlen_shapes(dev, lens, sal_frac, H, Hkv):
    """Column-sparse attention where the salient keys fill several groups per key block, and
    across the sequence length where the kernel switches from the two-pass to the single-pass
    path."""
    ops = _ops()
    print(f"[colsparse shapes] lens={lens} sal_frac={sal_frac}", flush=True)
    cs = _colsparse_case(5, H, Hkv, True, lens=lens, sal_frac=sal_frac)
    Tq = cs["q"].shape[0]
    _, st0, _ = ref.attention_sparse_varlen(cs["q"], cs["k"], cs["dv"], cs["c"], cs["o_sal"], cs["cu_q"],
                                            cs["cu_k"], cs["idx_q"], 0.99)
    cos = ref.cosine_from_stats(st0).numpy()
    tau = float(np.median(cos))
    want_o, want_st, want_m = ref.attention_sparse_varlen(cs["q"], cs["k"], cs["dv"], cs["c"], cs["o_sal"],
                                                          cs["cu_q"], cs["cu_k"], cs["idx_q"], tau)
    t = lambda a: torch.as_tensor(a).to(dev)
    stats = torch.zeros(Tq, 3, dtype=torch.float32, device=dev)
    mask = torch.empty(Tq, dtype=torch.bool, device=dev)
    o = ops.attention_sparse_varlen(t(cs["q"]), t(cs["k"]), t(cs["dv"]), t(cs["c"]), t(cs["o_sal"]), t(cs["cu_q"]),
                                    t(cs["cu_k"]), cs["maxq"], cs["maxk"], Tq, t(cs["cu_s"]), t(cs["idx_q"]), stats,
                                    mask, tau, True, t(cs["idx_k"]))
    assert_bf16_close(o, want_o, what="column-sparse output")
    assert torch.equal(o.cpu()[torch.from_numpy(cs["idx_q"]).long()], cs["o_sal"])
    torch.testing.assert_close(stats.cpu(), want_st, rtol=1e-4, atol=1e-2)
    excluded = assert_mask_equal(mask.cpu().numpy(), want_m.numpy(), cos, tau)
    assert excluded < Tq // 20


# ---------------------------------------------------------------------------------------
# FFN / MoE
# ---------------------------------------------------------------------------------------
# (400, 3584, 512): Dream's hidden size, whose 14 down-projection column tiles leave tile counts
# below the CU count that are not a multiple of 8; (600, 256, 11008) and (1600, 1024, 1536): the
# down projection (both) and the gate_up GEMM (the latter) take the M-split tile walk
@pytest.mark.parametrize("M,hidden,inter", [(77, 256, 512), (300, 512, 384), (600, 256, 11008), (920, 4096, 1024),
                                            (1500, 1024, 2048), (400, 3584, 512), (1600, 1024, 1536)])
def test_swiglu_ffn_gathered(dev, M, hidden, inter):
    ops = _ops()
    g = _gen(M)
    T = M * 3 + 5
    x = _randn(g, T, hidden)
    # fan-in scaled weights keep the outputs O(1), where a bf16 ulp is below the 2e-2 bar
    wgu = _randn(g, 2 * inter, hidden, scale=hidden ** -0.5)
    wd = _randn(g, hidden, inter, scale=inter ** -0.5)
    rows = torch.from_numpy(np.sort(np.random.default_rng(M).choice(T, size=M, replace=False))).to(torch.int32)
    y = ops.swiglu_ffn(x.to(dev), wgu.to(dev), wd.to(dev), rows_idx=rows.to(dev))
    want = ref.swiglu_ffn(x[rows.long()], wgu, wd)
    assert_bf16_close(y, want.to(BF), what="SwiGLU FFN")
    # in-place scatter epilogue into a cache
    cache = torch.zeros(T + 10, hidden, dtype=BF, device=dev)
    dest = torch.arange(M, dtype=torch.int64) * 2 + 3
    ops.swiglu_ffn(x.to(dev), wgu.to(dev), wd.to(dev), rows_idx=rows.to(dev), out=cache, out_rows=dest.to(dev))
    assert torch.equal(cache.cpu()[dest], y.cpu())
    untouched = torch.ones(T + 10, dtype=torch.bool)
    untouched[dest] = False
    assert (cache.cpu()[untouched] == 0).all()


@pytest.mark.parametrize("M,hidden,inter", [(2048, 512, 1024), (2500, 1024, 2048)])
def test_swiglu_ffn_dense_library_path(dev, M, hidden, inter):
    """A dense FFN of at least DENSE_FFN_LIBRARY_ROWS rows (the full step) runs the library GEMMs
    around dyllm_silu_and_mul: the same oracle bar as the fused kernels, and within the bf16 bound
    of the fused kernels' result on the same rows."""
    ops = _ops()
    assert M >= ops.DENSE_FFN_LIBRARY_ROWS
    print(f"[ffn dense] M={M} hidden={hidden} inter={inter}", flush=True)
    g = _gen(M + 1)
    x = _randn(g, M, hidden)
    wgu = _randn(g, 2 * inter, hidden, scale=hidden ** -0.5)
    wd = _randn(g, hidden, inter, scale=inter ** -0.5)
    xd, wgud, wdd = x.to(dev), wgu.to(dev), wd.to(dev)
    y = ops.swiglu_ffn(xd, wgud, wdd)
    assert_bf16_close(y, ref.swiglu_ffn(x, wgu, wd).to(BF), what="dense SwiGLU FFN (library GEMMs)")
    fused = ops.ffn_down(ops.ffn_gate_up(xd, wgud), wdd)
    assert_bf16_close(y, fused, what="library vs fused FFN")


def test_moe_gate_align_experts(dev):
    ops = _ops()
    g = _gen(21)
    T, hidden, E, top_k, inter = 300, 256, 64, 8, 128
    x = _randn(g, T, hidden)
    wr = _randn(g, E, hidden, scale=0.1)
    w, ids = ops.moe_gate(x.to(dev), wr.to(dev), top_k)
    w_ref, ids_ref = ref.moe_gate(x, wr, top_k)
    assert torch.equal(ids.cpu(), ids_ref)
    assert_routing_weights(w, w_ref)
    sorted_ids, tile_e, npp = ops.moe_align_block_size(ids, 128, E)
    s_ref, e_ref, n_ref = ref.moe_align_block_size(ids_ref.numpy(), 128, E)
    assert int(npp.item()) == n_ref
    assert np.array_equal(sorted_ids.cpu().numpy()[:n_ref], s_ref)
    assert np.array_equal(tile_e.cpu().numpy()[:n_ref // 128], e_ref)
    w1 = _randn(g, E, 2 * inter, hidden, scale=0.05)
    w2 = _randn(g, E, hidden, inter, scale=0.05)
    out = ops.fused_experts(x.to(dev), w1.to(dev), w2.to(dev), w_ref.to(dev), ids_ref.to(dev))
    want = ref.naive_experts(x, w1, w2, w_ref, ids_ref)
    assert_bf16_close(out, want.to(BF), what="fused experts")


def test_moe_gathered_rows_match_compacted(dev):
    """Router and experts reading the salient rows in place (rows_idx) give bit-identical routing
    and outputs to the same calls on the gathered rows (gather_rows_2D, util.py:19-36), and write
    only the destination rows."""
    ops = _ops()
    g = _gen(22)
    T_all, hidden, E, top_k, inter = 500, 256, 64, 8, 128
    x_all = _randn(g, T_all, hidden).to(dev)
    rows = torch.randperm(T_all, generator=g)[:173].to(torch.int32).to(dev)
    wr = _randn(g, E, hidden, scale=0.1).to(dev)
    w1 = _randn(g, E, 2 * inter, hidden, scale=0.05).to(dev)
    w2 = _randn(g, E, hidden, inter, scale=0.05).to(dev)
    x = x_all[rows.long()].contiguous()
    w, ids = ops.moe_gate(x, wr, top_k)
    wg, idg = ops.moe_gate(x_all, wr, top_k, rows_idx=rows)
    assert torch.equal(ids, idg) and torch.equal(w, wg)
    dest = torch.randperm(T_all + 50, generator=g)[:173].to(dev)
    want = torch.zeros(T_all + 50, hidden, dtype=BF, device=dev)
    ops.fused_experts(x, w1, w2, w, ids, out=want, out_rows=dest)
    got = torch.zeros_like(want)
    ops.fused_experts(x_all, w1, w2, w, ids, out=got, out_rows=dest, rows_idx=rows)
    assert torch.equal(got, want)


@pytest.mark.parametrize("T,hidden,E,top_k,renorm", [(1, 48, 8, 2, False), (33, 48, 8, 2, True), (70, 272, 13, 4, False),
                                                     (257, 2048, 64, 8, True)])
def test_moe_gate_shapes(dev, T, hidden, E, top_k, renorm):
    """Router over token counts that leave a partial 32-token tile, hidden sizes whose 16-wide
    steps do not divide evenly over the 8 slices of the hidden dimension (48: some slices empty),
    expert counts below 64 and renormalised weights: the expert sets equal the oracle's wherever
    its k-th and (k+1)-th probabilities are separated, and the weights agree within one bf16 ulp."""
    ops = _ops()
    g = _gen(60 + T)
    x = _randn(g, T, hidden)
    wr = _randn(g, E, hidden, scale=hidden ** -0.5)
    w, ids = ops.moe_gate(x.to(dev), wr.to(dev), top_k, renormalize=renorm)
    w_ref, ids_ref = ref.moe_gate(x, wr, top_k, renormalize=renorm)
    probs = torch.softmax(x.float() @ wr.float().t(), dim=-1)
    top = probs.topk(min(top_k + 1, E), dim=-1).values
    clear = (top[:, top_k - 1] - top[:, top_k]) > 1e-5 if top_k < E else torch.ones(T, dtype=torch.bool)
    assert clear.float().mean() > 0.9
    assert torch.equal(ids.cpu()[clear], ids_ref[clear])
    assert_routing_weights(w.cpu()[clear], w_ref[clear])


def test_moe_align_clamps_out_of_range_ids(dev):
    """Expert ids outside [0, E) are clamped on the device (never index past the LDS tables):
    the result equals the alignment of the clamped ids."""
    ops = _ops()
    E = 8
    ids = torch.tensor([[3, -5], [99, 0], [7, 8], [1, -1]], dtype=torch.int32)
    sorted_ids, tile_e, npp = ops.moe_align_block_size(ids.to(dev), 4, E)
    s_ref, e_ref, n_ref = ref.moe_align_block_size(ids.clamp(0, E - 1).numpy(), 4, E)
    assert int(npp.item()) == n_ref
    assert np.array_equal(sorted_ids.cpu().numpy()[:n_ref], s_ref)
    assert np.array_equal(tile_e.cpu().numpy()[:n_ref // 4], e_ref)


@pytest.mark.parametrize("S,E,bm,skew", [(0, 8, 4, 0.0), (1, 64, 128, 0.0), (511, 64, 16, 0.0), (513, 7, 32, 3.0),
                                          (5000, 64, 128, 2.0), (29488, 64, 128, 0.5), (70001, 13, 64, 1.0)])
def test_moe_align_workgroups(dev, S, E, bm, skew):
    """Alignment over 1 to 64 workgroups (chunks of >= 512 slots; uneven last chunks, experts with
    no slots, skewed loads): the buckets equal the oracle's, the padding and the tail past the last
    bucket hold the sentinel, and every tile past the last bucket is assigned expert 0."""
    ops = _ops()
    g = _gen(40 + S)
    logits = torch.randn(E, generator=g) * skew
    p = torch.softmax(logits, 0)
    ids = torch.multinomial(p, S, replacement=True, generator=g).to(torch.int32) if S else torch.zeros(0, dtype=torch.int32)
    ids2 = ids.reshape(-1, 1)
    sorted_ids, tile_e, npp = ops.moe_align_block_size(ids2.to(dev), bm, E)
    s_ref, e_ref, n_ref = ref.moe_align_block_size(ids2.numpy(), bm, E)
    got_s, got_e = sorted_ids.cpu().numpy(), tile_e.cpu().numpy()
    assert int(npp.item()) == n_ref
    assert np.array_equal(got_s[:n_ref], s_ref)
    assert np.array_equal(got_e[:n_ref // bm], e_ref)
    assert (got_s[n_ref:] == S).all()
    assert (got_e[n_ref // bm:] == 0).all()


def test_attention_kernel_info(dev):
    """attention.cpp:205-208 mirror: [regs, local_bytes, static_smem, dynamic_smem, tb_size,
    max_active_blocks_per_sm, block_q, block_k, d_split, ok]."""
    info = _ops().attention_kernel_info(128)
    assert len(info) == 10
    regs, local, smem, dyn, tb, blocks, bq, bk, dsplit, ok = info
    assert 0 < regs <= 512 and tb == 256 and bq == 128 and bk == 64 and ok == 1
    assert 0 < smem <= 160 * 1024 and blocks >= 1 and local >= 0
    assert _ops().attention_kernel_info(96)[-1] == 0
