"""Config 0 on the GPU: one LLaDA-style layer's saliency hot path at its exact workload
(B = 1, 128 prompt + 384 response rows, hidden 4096 = 32 heads x 128, SwiGLU 12288, weights
N(0, 0.02), step-1 context ~ N(0, 1), step 2 = step 1 + Gaussian noise of sigma = 0.5 x row RMS on
a uniformly chosen 10% of the response rows, tau = 0.99), each stage against the CPU oracle:
saliency -> compaction -> gathered SwiGLU FFN -> partial attention of the salient queries against
the full K/V. Known answer: the salient set is exactly the perturbed rows. Then the whole fused
sparse step at the same shape with the known answer carried through attention."""
import math

import numpy as np
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close, assert_mask_equal

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
P, R, HID, H, D, INTER, TAU = 128, 384, 4096, 32, 128, 12288, 0.99


def _workload(seed=0):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    c1 = torch.randn(R, HID, generator=g)
    pert = np.sort(rng.choice(R, size=int(round(0.10 * R)), replace=False))
    c2 = c1.clone()
    rms = c1[pert].pow(2).mean(-1, keepdim=True).sqrt()
    c2[pert] += 0.5 * rms * torch.randn(len(pert), HID, generator=g)
    return g, c1.to(BF), c2.to(BF), pert


def test_config0_stages(dev):
    from dyllm_amd import ops

    print("[config0] stages", flush=True)
    g, c1, c2, pert = _workload(0)
    # saliency pass + tau test: the known answer and the oracle
    stats, mask = ops.saliency_stats(c2.to(dev), c1.to(dev), TAU)
    torch.cuda.synchronize()
    got_mask = mask.cpu().numpy()
    assert np.array_equal(np.nonzero(got_mask)[0], pert)
    want_st = ref.saliency_stats(c2.float(), c1.float())
    want_m = ref.cosine_mask(want_st, TAU).numpy()
    assert_mask_equal(got_mask, want_m, ref.cosine_from_stats(want_st).numpy(), TAU)
    assert torch.allclose(stats.cpu(), want_st, rtol=1e-4, atol=1e-2)
    cos = ref.cosine_from_stats(stats.cpu()).numpy()
    assert np.all(np.abs(cos[pert] - 1 / math.sqrt(1.25)) < 0.03)
    # compaction (+ the K-space rows of the Q-pruned step): bit-exact
    cu_q = torch.tensor([0, R], dtype=torch.int32)
    cu_p = torch.tensor([0, P], dtype=torch.int32)
    res = ops.salient_compact(mask, cu_q.to(dev), cu_p.to(dev))
    idx64, idx32, idx_k, cu_sal = res.trimmed()
    n = len(pert)
    assert res.n() == n
    idx_ref, cu_ref = ref.compact(got_mask, cu_q.numpy())
    assert np.array_equal(idx64.cpu().numpy(), idx_ref) and np.array_equal(cu_sal.cpu().numpy(), cu_ref)
    assert np.array_equal(idx_k.cpu().numpy(), ref.fused_offset(idx_ref, cu_p.numpy(), cu_ref))
    assert np.array_equal(idx_k.cpu().numpy(), pert + P)
    # gathered SwiGLU FFN over the salient rows, weights N(0, 0.02)
    wgu = (0.02 * torch.randn(2 * INTER, HID, generator=g)).to(BF)
    wd = (0.02 * torch.randn(HID, INTER, generator=g)).to(BF)
    y = ops.swiglu_ffn(c2.to(dev), wgu.to(dev), wd.to(dev), rows_idx=idx32)
    want_y = ref.swiglu_ffn(c2[torch.from_numpy(pert)], wgu, wd)
    # outputs reach |y| ~ 8 at this weight scale, where one bf16 ulp is 0.031: the bar is the
    # relative one plus one output ulp of the largest value
    assert_bf16_close(y, want_y.to(BF), max_abs=2 ** (math.floor(math.log2(want_y.abs().max().item())) - 7),
                      what="config-0 SwiGLU")
    # partial attention: the salient query rows against the full 512-row K/V
    q = torch.randn(P + R, H, D, generator=g).to(BF)
    k = torch.randn(P + R, H, D, generator=g).to(BF)
    v = torch.randn(P + R, H, D, generator=g).to(BF)
    o = ops.flash_attn_varlen_func(q.to(dev), k.to(dev), v.to(dev), torch.tensor([0, n], dtype=torch.int32, device=dev),
                                   torch.tensor([0, P + R], dtype=torch.int32, device=dev), n, P + R,
                                   q_rows=idx_k.to(torch.int32))
    want_o = ref.flash_attn_varlen(q[torch.from_numpy(pert + P)], k, v, [0, n], [0, P + R])
    assert_bf16_close(o, want_o, what="config-0 partial attention")


@pytest.mark.parametrize("noalloc", [False, True])
def test_config0_fused_step_known_answer(dev, noalloc):
    """The fused sparse step (Q-pruned) at config-0 shape: each response query is a scaled copy of
    its own key (one-hot attention), the previous salient set is 20% of the response rows, and the
    V rows of half of it (10% of the responses) move by sigma = 0.5 x row RMS. The next salient set
    must be exactly those rows, the step's outputs must match the oracle, and the V and context
    caches must hold the new rows."""
    from dyllm_amd import ops

    print(f"[config0] fused step noalloc={noalloc}", flush=True)
    g = torch.Generator().manual_seed(2024)
    rng = np.random.default_rng(2024)
    k = torch.randn(P + R, H, D, generator=g).to(BF)
    q = (4.0 * k[P:].float()).to(BF)
    v_old = torch.randn(P + R, H, D, generator=g).to(BF)
    sal = np.sort(rng.choice(R, size=77, replace=False))
    pert = np.sort(rng.choice(sal, size=38, replace=False))
    v_new = v_old[P + sal].float()
    rms = v_new.flatten(1).pow(2).mean(-1).sqrt()[:, None, None]
    is_p = torch.as_tensor(np.isin(sal, pert))
    v_new[is_p] += 0.5 * rms[is_p] * torch.randn(int(is_p.sum()), H, D, generator=g)
    v_new = v_new.to(BF)
    cu_q, cu_k, cu_p = np.array([0, R]), np.array([0, P + R]), np.array([0, P])
    c_old = ref.flash_attn_varlen(q, k, v_old, cu_q, cu_k)
    want = ref.sparse_attention_step(q, k, v_new, v_old, c_old, cu_q, cu_k, np.array([0, len(sal)]), sal, P + sal,
                                     cu_p, TAU)
    assert want["idx_salient_row"].tolist() == pert.tolist()

    i32 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int32, device=dev)
    i64 = lambda a: torch.as_tensor(np.asarray(a), dtype=torch.int64, device=dev)
    v_cache = v_old.reshape(P + R, H * D).to(dev)
    c_cache = torch.zeros(P + R, H * D, dtype=BF, device=dev)
    c_cache[P:] = c_old.reshape(R, H * D).to(dev)
    starts, seq_ids = i64([0]), i64([0])
    bufs = ops.StepBuffers(None, dev, R, P + R, 1, H, H, D, P + R, True)
    fn = ops.sparse_attention_step_noalloc if noalloc else ops.sparse_attention_step
    fn(bufs, q.to(dev), k.to(dev), v_cache, starts, v_new.to(dev), c_cache, starts, seq_ids, i32(cu_q), i32(cu_k),
       i32(cu_p), R, P + R, P + R, len(sal), len(sal), i32([0, len(sal)]), i32(sal), i64(P + sal), i32(P + sal),
       D ** -0.5, TAU)
    torch.cuda.synchronize()
    n = int(bufs.count.item())
    assert bufs.idx64[:n].cpu().tolist() == pert.tolist()
    assert bufs.idx_k64[:n].cpu().tolist() == (P + pert).tolist()
    assert bufs.cu_sal.cpu().tolist() == [0, len(pert)]
    assert_bf16_close(bufs.out, want["new_c"], what="config-0 step output")
    assert torch.equal(v_cache.cpu().view(P + R, H, D), want["v_cache"])
    assert torch.equal(c_cache[P:].cpu().view(R, H, D), bufs.out.cpu())
