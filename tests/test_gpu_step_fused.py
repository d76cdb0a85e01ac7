"""GPU checks of the fused sparse step's first launch (step_rows_kernel) and of the salient maps
the column-sparse tiles build from the compact lists:

* the salient lists may come in any order within a sequence (the first sparse layer takes them
  in the sampler's order, model_runner.py:208): a shuffled list gives bit-identical outputs,
  caches and next salient set;
* ``Attention.forward(q, None, KvRows)`` -- the K/V epilogue (k_norm, RoPE, K-cache row) fused
  into the step, K read from its cache in place -- is bit-identical to the two-pass composition
  the reference runs (scatter of the rotated keys, llada.py:136-146, then Attention.forward with
  the packed K and the v rows, attention.py:64-178), including kv rows addressed through an index.

Both paths run the same kernels downstream, so equality is exact."""
import numpy as np
import pytest
import torch

from tests.test_gpu_layer import _setup

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _ctx(s, dev, idx_q, idx_k, q_pruned, tau=0.99):
    from dyllm_amd.utils.context import set_context

    t = s["t"]
    s["attn"].threshold = tau
    return set_context(False, cu_seqlens_q=t(s["cu_q"]), cu_seqlens_q_cpu=s["cu_q"].tolist(),
                       cu_seqlens_k=t(s["cu_k"]), cu_seqlens_k_cpu=s["cu_k"].tolist(), cu_promptlens=t(s["cu_p"]),
                       max_seqlen_q=max(s["Lq"]), max_seqlen_k=max(s["Lk"]), context_lens_cpu=s["Lk"],
                       cu_salientlens=t(s["cu_s"]), idx_salient_row=t(idx_q, torch.long),
                       idx_salient_row_k=t(idx_k, torch.long) if q_pruned else None,
                       total_seqlen=s["Tq"], total_seqlen_k=s["Tk"])


def _result(s, ctx, new_c):
    attn = s["attn"]
    return dict(new_c=new_c.cpu(), v=attn.v_cache.cache.cpu(), c=attn.context_cache.cache.cpu(),
                idx=ctx.idx_salient_row.cpu(), cu=ctx.cu_salientlens.cpu(),
                idx_k=None if ctx.idx_salient_row_k is None else ctx.idx_salient_row_k.cpu())


def _assert_same(a, b):
    for key in a:
        if a[key] is None:
            assert b[key] is None, key
        else:
            assert torch.equal(a[key], b[key]), key


def _shuffle_within(s, seed):
    """A per-sequence permutation of the salient list entries (Q and K lists together)."""
    rng = np.random.default_rng(seed)
    perm = []
    for b in range(len(s["cu_s"]) - 1):
        seg = np.arange(s["cu_s"][b], s["cu_s"][b + 1])
        perm += rng.permutation(seg).tolist()
    return np.asarray(perm, dtype=np.int64)


@pytest.mark.parametrize("q_pruned,sal_counts", [(True, None), (False, None), (True, [80, 200, 64])])
def test_unsorted_salient_lists_give_identical_step(dev, q_pruned, sal_counts):
    print(f"[step order] q_pruned={q_pruned} sal_counts={sal_counts}", flush=True)
    out = []
    for shuffled in (False, True):
        s = _setup(dev, q_pruned, sal_counts=sal_counts, seed=4)
        perm = _shuffle_within(s, 7) if shuffled else np.arange(len(s["idx_q"]))
        ctx = _ctx(s, dev, s["idx_q"][perm], s["idx_k"][perm], q_pruned)
        new_c = s["attn"](s["q"].to(dev), s["k_new"].to(dev), s["v_new"][torch.from_numpy(perm)].to(dev))
        out.append(_result(s, ctx, new_c))
    _assert_same(out[0], out[1])


@pytest.mark.parametrize("q_pruned,k_norm,indexed", [(True, False, False), (True, True, True), (False, False, True)])
def test_kv_rows_epilogue_fused_into_step(dev, q_pruned, k_norm, indexed):
    from dyllm_amd import ops
    from dyllm_amd.engine.cache_manager import CacheManager
    from oracle import dyllm_oracle as ref

    print(f"[step kv] q_pruned={q_pruned} k_norm={k_norm} indexed={indexed}", flush=True)
    out = []
    for fused in (False, True):
        s = _setup(dev, q_pruned, seed=9)
        md = s["md"]
        g = torch.Generator().manual_seed(21)
        Hkv, n = s["Hkv"], len(s["idx_k"])
        kvs = Hkv * 128
        # the K cache before this step, slab rows of the running sequences at scattered starts
        k_cache = CacheManager(kvs, device=dev)
        for sid in md.running_seqs[::-1]:   # allocation order differs from batch order: no packed view
            b = md.running_seqs.index(sid)
            k_cache.reset_seq(s["k_new"][s["cu_k"][b]:s["cu_k"][b + 1]].flatten(1).to(dev), sid)
        # projection output of the salient rows: [k | v]; k before its epilogue
        kv = torch.cat([(torch.randn(n, kvs, generator=g) * 1.5).to(BF), s["v_new"].flatten(1)], dim=1)
        rows = np.arange(n)
        if indexed:   # rows addressed through kv_rows (a larger buffer in another order)
            rows = np.random.default_rng(3).permutation(n + 5)[:n]
            big = torch.zeros(n + 5, 2 * kvs, dtype=BF)
            big[torch.from_numpy(rows)] = kv
            kv_dev = big.to(dev)
        else:
            kv_dev = kv.to(dev)
        positions = torch.randint(0, 2048, (s["Tq"],), generator=g).to(dev)
        cos, sin = (x.to(dev) for x in ref.rope_tables(128, 4096, 10000.0))
        kn = (1 + 0.2 * torch.randn(128, generator=g)).to(BF).to(dev) if k_norm else None
        ctx = _ctx(s, dev, s["idx_q"], s["idx_k"], q_pruned)
        idx32 = ctx.idx_salient_row_i32
        if fused:
            v = k_cache.kv_rows(kv_dev, Hkv, positions, cos, sin, idx32,
                                kv_rows=torch.from_numpy(rows).to(dev) if indexed else None, k_norm_weight=kn)
            new_c = s["attn"](s["q"].to(dev), None, v)
        else:
            src = kv_dev[torch.from_numpy(rows).to(dev)] if indexed else kv_dev
            kidx = ctx.idx_salient_row_k if q_pruned else ctx.idx_salient_row
            v = k_cache.scatter_kv_rope(md.running_seqs_tensor, kidx, src, Hkv, positions, cos, sin, idx32,
                                        k_norm_weight=kn)
            k_full = k_cache.get_seqs(md.running_seqs_tensor, md.running_seqs).view(-1, Hkv, 128)
            new_c = s["attn"](s["q"].to(dev), k_full, v)
        r = _result(s, ctx, new_c)
        r["k"] = k_cache.cache.cpu()
        out.append(r)
    _assert_same(out[0], out[1])
