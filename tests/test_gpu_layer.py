"""GPU parity of the product path at layer level: ``Attention.forward`` (sparse Q-pruned and
refresh steps, with the caches and the context mutation) and the fused gathered FFN with its
cache scatter, against the oracle's end-to-end restatement of attention.py:64-178."""
import numpy as np
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close, assert_mask_equal

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _setup(dev, q_pruned, H=4, Hkv=2, lens=((48, 80), (16, 200), (64, 64)), seed=0, tau=None, sal_counts=None):
    from dyllm_amd.engine.cache_manager import CacheManager
    from dyllm_amd.model_executor.layers.attention import Attention
    from dyllm_amd.utils.context import set_context
    from dyllm_amd.utils.metadata import get_metadata

    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    D = 128
    B = len(lens)
    Lk = [p + r for p, r in lens]
    Lq = [r if q_pruned else p + r for p, r in lens]
    cu_k = np.concatenate([[0], np.cumsum(Lk)]).astype(np.int32)
    cu_q = np.concatenate([[0], np.cumsum(Lq)]).astype(np.int32)
    cu_p = np.concatenate([[0], np.cumsum([p for p, _ in lens])]).astype(np.int32)
    Tk, Tq = int(cu_k[-1]), int(cu_q[-1])
    md = get_metadata()
    md.running_seqs = [5, 2, 9][:B]
    md.running_seqs_tensor = torch.tensor(md.running_seqs, dtype=torch.long, device=dev)
    md.finished_seqs = []
    t = lambda a, dt=torch.int32: torch.as_tensor(np.asarray(a)).to(dt).to(dev)
    # dense step: fill the caches
    set_context(True, cu_seqlens_q=t(cu_k), cu_seqlens_q_cpu=cu_k.tolist(), cu_seqlens_k=t(cu_k),
                cu_seqlens_k_cpu=cu_k.tolist(), max_seqlen_q=max(Lk), max_seqlen_k=max(Lk), context_lens_cpu=Lk,
                total_seqlen=Tk, total_seqlen_k=Tk)
    attn = Attention(H, D, D ** -0.5, Hkv, 0.99, device=dev)
    q_all = torch.randn(Tk, H, D, generator=g).to(BF)
    k_all = torch.randn(Tk, Hkv, D, generator=g).to(BF)
    v_all = torch.randn(Tk, Hkv, D, generator=g).to(BF)
    o_full = attn(q_all.to(dev), k_all.to(dev), v_all.to(dev))
    # salient rows of this step (response rows), new V/K rows
    idx_q, idx_k, cu_s = [], [], [0]
    for b, (p, r) in enumerate(lens):
        n_b = max(1, r // 6) if sal_counts is None else sal_counts[b]
        sel = np.sort(rng.choice(r, size=n_b, replace=False))
        idx_k += (cu_k[b] + p + sel).tolist()
        idx_q += ((cu_q[b] + sel) if q_pruned else (cu_q[b] + p + sel)).tolist()
        cu_s.append(len(idx_q))
    idx_k = np.asarray(idx_k, dtype=np.int64)
    v_new = (v_all[idx_k].float() + 0.5 * torch.randn(len(idx_k), Hkv, D, generator=g)).to(BF)
    k_new = k_all.clone()
    k_new[idx_k] = (k_all[idx_k].float() + 0.5 * torch.randn(len(idx_k), Hkv, D, generator=g)).to(BF)
    resp = np.concatenate([np.arange(cu_k[b] + lens[b][0], cu_k[b + 1]) for b in range(B)]) if q_pruned \
        else np.arange(Tk)
    q = q_all[resp]
    return dict(attn=attn, q=q, k_new=k_new, v_new=v_new, v_old=v_all, o_full=o_full.cpu(), cu_q=cu_q, cu_k=cu_k,
                cu_p=cu_p, cu_s=np.asarray(cu_s), idx_q=np.asarray(idx_q, dtype=np.int64), idx_k=idx_k, resp=resp, Tq=Tq, Tk=Tk,
                t=t, md=md, H=H, Hkv=Hkv, Lq=Lq, Lk=Lk)


# sequences longer than one 4096-key chunk of the two-pass column-sparse tiles (ragged: 2 and 3
# chunks) beside a short one
LONG = ((256, 4200), (64, 8300), (16, 300))


@pytest.mark.parametrize("q_pruned,sal_counts,lens", [(True, None, None), (False, None, None), (True, [0, 7, 64], None),
                                                       (False, [0, 0, 0], None), (True, [80, 200, 64], None),
                                                       (True, [1, 0, 1], None), (True, [300, 500, 10], LONG),
                                                       (False, [120, 0, 64], LONG)])
def test_attention_forward_sparse_step(dev, q_pruned, sal_counts, lens):
    """Sparse step at layer level; the salient sets include a sequence with no salient row, no
    salient row at all, every response row salient, and single rows; sequences of up to 8364 keys
    (several key chunks of the two-pass column-sparse tiles)."""
    from dyllm_amd.utils.context import set_context

    print(f"[layer] q_pruned={q_pruned} sal_counts={sal_counts} lens={lens}", flush=True)
    s = _setup(dev, q_pruned, sal_counts=sal_counts, **({"lens": lens} if lens else {}))
    t, md = s["t"], s["md"]
    # oracle inputs: packed caches as the reference's get_seqs / get_seqs_block return them
    c_old = s["o_full"][torch.from_numpy(s["resp"])] if q_pruned else s["o_full"]
    # pick tau in the middle of the cosine distribution so the set is non-trivial
    probe = ref.sparse_attention_step(s["q"], s["k_new"], s["v_new"], s["v_old"], c_old, s["cu_q"], s["cu_k"],
                                      s["cu_s"], s["idx_q"], s["idx_k"] if q_pruned else None, s["cu_p"], 0.99)
    cos = ref.cosine_from_stats(probe["stats"]).numpy()
    tau = float(np.median(cos))
    want = ref.sparse_attention_step(s["q"], s["k_new"], s["v_new"], s["v_old"], c_old, s["cu_q"], s["cu_k"],
                                     s["cu_s"], s["idx_q"], s["idx_k"] if q_pruned else None, s["cu_p"], tau)
    attn = s["attn"]
    attn.threshold = tau
    ctx = set_context(False, cu_seqlens_q=t(s["cu_q"]), cu_seqlens_q_cpu=s["cu_q"].tolist(),
                      cu_seqlens_k=t(s["cu_k"]), cu_seqlens_k_cpu=s["cu_k"].tolist(), cu_promptlens=t(s["cu_p"]),
                      max_seqlen_q=max(s["Lq"]), max_seqlen_k=max(s["Lk"]), context_lens_cpu=s["Lk"],
                      cu_salientlens=t(s["cu_s"]), idx_salient_row=t(s["idx_q"], torch.long),
                      idx_salient_row_k=t(s["idx_k"], torch.long) if q_pruned else None,
                      total_seqlen=s["Tq"], total_seqlen_k=s["Tk"])
    new_c = attn(s["q"].to(dev), s["k_new"].to(dev), s["v_new"].to(dev))
    assert_bf16_close(new_c, want["new_c"], what="new context")
    # context mutation for the next layer: bit-exact salient set outside the tau band
    got_mask = np.zeros(s["Tq"], bool)
    got_mask[ctx.idx_salient_row.cpu().numpy()] = True
    assert_mask_equal(got_mask, want["mask"].numpy(), cos, tau)
    if not np.any(np.abs(cos - tau) <= 1e-6):
        assert np.array_equal(ctx.idx_salient_row.cpu().numpy(), want["idx_salient_row"])
        assert np.array_equal(ctx.cu_salientlens.cpu().numpy(), want["cu_salientlens"])
        if q_pruned:
            assert np.array_equal(ctx.idx_salient_row_k.cpu().numpy(), want["idx_salient_row_k"])
    assert (ctx.idx_salient_row_k is None) == (not q_pruned)
    # caches: V cache holds the new rows; the context cache holds the new context rows
    v_cache = attn.v_cache.cache.cpu().view(-1, s["Hkv"], 128)
    assert torch.equal(v_cache, want["v_cache"])
    ctx_rows = attn.context_cache.cache.cpu().view(-1, s["H"], 128)[torch.from_numpy(s["resp"])]
    assert torch.equal(ctx_rows, new_c.cpu())


def test_fused_ffn_scatter_matches_reference_mlp(dev):
    """LLaDAMLP.forward_salient (gather inside the GEMM, scatter into the FFN cache, read back of
    all queried rows) == gather_rows_2D -> SwiGLU -> MLPcache (llada.py:184-186,
    mlp_cache_manage.py:24-40)."""
    from dyllm_amd.model_executor.models.llada import LLaDAMLP
    from dyllm_amd.utils.context import set_context
    from dyllm_amd.utils.metadata import get_metadata

    g = torch.Generator(device=dev).manual_seed(3)
    B, P, R, hid, inter = 3, 20, 60, 256, 384
    L = P + R
    md = get_metadata()
    md.running_seqs = [0, 1, 2]
    md.running_seqs_tensor = torch.arange(3, device=dev)
    md.finished_seqs = []
    cu_k = [i * L for i in range(B + 1)]
    cu_q = [i * R for i in range(B + 1)]
    i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)
    set_context(True, cu_seqlens_q=i32(cu_k), cu_seqlens_q_cpu=cu_k, cu_seqlens_k=i32(cu_k), cu_seqlens_k_cpu=cu_k,
                max_seqlen_q=L, max_seqlen_k=L, context_lens_cpu=[L] * B, total_seqlen=B * L, total_seqlen_k=B * L)
    mlp = LLaDAMLP(hid, inter, device=dev, gen=g)
    with torch.no_grad():
        mlp.gate_up_proj.data = (torch.randn(2 * inter, hid, device=dev) * hid ** -0.5).to(BF)
        mlp.down_proj.data = (torch.randn(hid, inter, device=dev) * inter ** -0.5).to(BF)
    x_full = torch.randn(B * L, hid, device=dev).to(BF)
    cache0 = mlp(x_full).cpu()  # full step: FFN of all rows into the cache
    rng = np.random.default_rng(0)
    idx_q = np.sort(rng.choice(B * R, size=40, replace=False))
    idx_k = (idx_q // R) * L + P + idx_q % R
    set_context(False, cu_seqlens_q=i32(cu_q), cu_seqlens_q_cpu=cu_q, cu_seqlens_k=i32(cu_k), cu_seqlens_k_cpu=cu_k,
                max_seqlen_q=R, max_seqlen_k=L, context_lens_cpu=[L] * B, total_seqlen=B * R, total_seqlen_k=B * L,
                idx_salient_row=torch.from_numpy(idx_q).to(dev), idx_salient_row_k=torch.from_numpy(idx_k).to(dev))
    h = torch.randn(B * R, hid, device=dev).to(BF)
    out = mlp.forward_salient(h).cpu()
    y = ref.swiglu_ffn(h.cpu()[torch.from_numpy(idx_q)], mlp.gate_up_proj.cpu(), mlp.down_proj.cpu()).to(BF)
    resp = np.concatenate([np.arange(b * L + P, (b + 1) * L) for b in range(B)])
    want = cache0[torch.from_numpy(resp)].clone()
    want[torch.from_numpy(idx_q)] = y
    assert_bf16_close(out, want, what="FFN cache rows")
    # untouched rows are bit-identical to the previous step's cache
    keep = np.setdiff1d(np.arange(B * R), idx_q)
    assert torch.equal(out[torch.from_numpy(keep)], want[torch.from_numpy(keep)])


@pytest.mark.parametrize("L", [100, 700])
def test_mlp_full_step_dense_rows(dev, L):
    """Full-step FFN over all rows (3 x 100 and 3 x 700 rows) through LLaDAMLP.forward: matches
    the fp32 oracle when read back from the FFN cache, as the full step returns it."""
    from dyllm_amd.model_executor.models.llada import LLaDAMLP
    from dyllm_amd.utils.context import set_context
    from dyllm_amd.utils.metadata import get_metadata

    print(f"[mlp full] rows={3 * L}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    B, hid, inter = 3, 256, 384
    T = B * L
    md = get_metadata()
    md.running_seqs = [0, 1, 2]
    md.running_seqs_tensor = torch.arange(3, device=dev)
    md.finished_seqs = []
    cu = [i * L for i in range(B + 1)]
    i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)
    set_context(True, cu_seqlens_q=i32(cu), cu_seqlens_q_cpu=cu, cu_seqlens_k=i32(cu), cu_seqlens_k_cpu=cu,
                max_seqlen_q=L, max_seqlen_k=L, context_lens_cpu=[L] * B, total_seqlen=T, total_seqlen_k=T)
    mlp = LLaDAMLP(hid, inter, device=dev, gen=g)
    with torch.no_grad():
        mlp.gate_up_proj.data = (torch.randn(2 * inter, hid, device=dev, generator=g) * hid ** -0.5).to(BF)
        mlp.down_proj.data = (torch.randn(hid, inter, device=dev, generator=g) * inter ** -0.5).to(BF)
    x = torch.randn(T, hid, device=dev, generator=g).to(BF)
    y = mlp(x).cpu()
    want = ref.swiglu_ffn(x.cpu(), mlp.gate_up_proj.cpu(), mlp.down_proj.cpu()).to(BF)
    assert_bf16_close(y, want, what="full-step FFN")
