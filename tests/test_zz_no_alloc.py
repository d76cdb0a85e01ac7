"""dyllm_sparse_attention_step_noalloc (workspace in the library's per-GPU scratch array) against
dyllm_sparse_attention_step (caller workspace): identical outputs, caches and next salient sets,
bit for bit, on two calls in a row -- the second with a smaller input -- plus the size limit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
D = 128


def _case(dev, seed, B, P, R, H, Hkv, n_per, q_pruned):
    g = torch.Generator(device=dev).manual_seed(seed)
    rng = np.random.default_rng(seed)
    L = P + R
    Tk = B * L
    Tq = B * R if q_pruned else Tk
    cu_k = np.arange(B + 1, dtype=np.int64) * L
    cu_q = np.arange(B + 1, dtype=np.int64) * (R if q_pruned else L)
    cu_p = np.arange(B + 1, dtype=np.int64) * P
    sel = [np.sort(rng.choice(R, size=n_per, replace=False)) for _ in range(B)]
    idx_k = np.concatenate([cu_k[b] + P + sel[b] for b in range(B)])
    idx_q = np.concatenate([cu_q[b] + (0 if q_pruned else P) + sel[b] for b in range(B)])
    rnd = lambda *s: torch.randn(*s, generator=g, device=dev).to(BF)
    i32 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int32, device=dev)
    i64 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int64, device=dev)
    return dict(
        B=B, Tq=Tq, Tk=Tk, H=H, Hkv=Hkv, L=L, R=R, n=len(idx_q), n_per=n_per,
        q=rnd(Tq, H, D), k=rnd(Tk, Hkv, D), v_cache=rnd(Tk, Hkv * D), v_new=rnd(len(idx_k), Hkv, D),
        c_cache=rnd(Tk, H * D), starts=i64(cu_k[:-1]), seq_ids=torch.arange(B, device=dev),
        cu_q=i32(cu_q), cu_k=i32(cu_k), cu_p=i32(cu_p) if q_pruned else None,
        cu_s=i32(np.arange(B + 1) * n_per), idx_q32=i32(idx_q), idx_k64=i64(idx_k), idx_k32=i32(idx_k),
        q_pruned=q_pruned)


def _run(c, fn, dev):
    from dyllm_amd import ops

    bufs = ops.StepBuffers(None, dev, c["Tq"], c["Tk"], c["B"], c["H"], c["Hkv"], D, c["L"], c["q_pruned"])
    v_cache, c_cache = c["v_cache"].clone(), c["c_cache"].clone()
    fn(bufs, c["q"], c["k"], v_cache, c["starts"], c["v_new"], c_cache, c["starts"], c["seq_ids"], c["cu_q"],
       c["cu_k"], c["cu_p"], c["R"] if c["q_pruned"] else c["L"], c["L"], c["Tk"], c["n"], c["n_per"], c["cu_s"],
       c["idx_q32"], c["idx_k64"], c["idx_k32"], D ** -0.5, 0.99)
    torch.cuda.synchronize()
    n = int(bufs.count.item())
    res = dict(out=bufs.out, stats=bufs.stats, mask=bufs.mask, v_cache=v_cache, c_cache=c_cache,
               idx64=bufs.idx64[:n], idx32=bufs.idx32[:n], cu_sal=bufs.cu_sal, count=bufs.count,
               host_meta=bufs.host_meta)
    if c["q_pruned"]:
        res.update(idx_k64=bufs.idx_k64[:n], idx_k32=bufs.idx_k32[:n])
    return {k: v.cpu().clone() for k, v in res.items()}


@pytest.mark.parametrize("q_pruned", [True, False])
def test_noalloc_step_matches_workspace_step(dev, q_pruned):
    from dyllm_amd import ops

    for call, shape in enumerate([(4, 96, 320, 8, 4, 40), (2, 64, 128, 8, 4, 9)]):
        B, P, R, H, Hkv, n_per = shape
        print(f"[no_alloc] call {call} q_pruned={q_pruned} B={B} P={P} R={R} H={H}/{Hkv} n_per={n_per}", flush=True)
        c = _case(dev, 100 + call, B, P, R, H, Hkv, n_per, q_pruned)
        want = _run(c, ops.sparse_attention_step, dev)
        got = _run(c, ops.sparse_attention_step_noalloc, dev)
        assert 0 < int(want["count"][0]) < c["Tq"]
        for name in want:
            assert torch.equal(got[name], want[name]), f"call {call}: {name} differs"


def test_noalloc_step_refuses_oversize(dev):
    from dyllm_amd import _lib, ops

    lib = _lib.load()
    cap = lib.dyllm_sparse_step_scratch_bytes()
    # config-4 shape (2 x 8192 rows, refresh) with every row salient needs more than the scratch holds
    need = lib.dyllm_sparse_step_workspace_bytes(2, 32, 32, D, 16384, 16384, 8192, 16384)
    assert need > cap
    c = _case(dev, 7, 1, 16, 48, 2, 2, 4, True)
    with pytest.raises(RuntimeError, match="scratch"):
        ops.sparse_attention_step_noalloc(
            ops.StepBuffers(None, dev, c["Tq"], c["Tk"], 1, 2, 2, D, c["L"], True), c["q"], c["k"],
            c["v_cache"], c["starts"], c["v_new"], c["c_cache"], c["starts"], c["seq_ids"], c["cu_q"], c["cu_k"],
            c["cu_p"], c["R"], c["L"], c["Tk"], 300_000, 4, c["cu_s"], c["idx_q32"], c["idx_k64"],
            c["idx_k32"], D ** -0.5, 0.99)
