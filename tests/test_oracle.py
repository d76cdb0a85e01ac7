"""Pins the CPU oracle (oracle/dyllm_oracle.py) before it is trusted as the checker: against the
reference's own known-answer test, against closed forms / library routines, against brute
force on tiny inputs, and against invariants chosen so that a plausible mistake (dropped term,
wrong sign or index, transposed operand, wrong rounding point) fails."""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dyllm_oracle as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BF = torch.bfloat16


def test_tau_known_answer_fixture():
    """The reference's additive-shard cosine test (tests/test_parallelism.py:34-44)."""
    with open(os.path.join(GOLDEN, "tau_known_answer.json")) as f:
        fx = json.load(f)
    stats = torch.tensor(fx["stats"], dtype=torch.float32)
    assert ref.cosine_mask(stats, fx["threshold"]).tolist() == fx["expected_mask"]
    # and it equals torch's cosine_similarity decision, as the reference test asserts
    old, new = torch.tensor(fx["old"]), torch.tensor(fx["new"])
    assert ref.cosine_mask(stats, fx["threshold"]).tolist() == (F.cosine_similarity(old, new, dim=-1) < 0.5).tolist()


def test_cosine_mask_clamps_and_orientation():
    # zero vectors: both norms clamp to 1e-8 -> cos = 0 -> salient for any positive tau
    s = torch.tensor([[0.0, 0.0, 0.0], [4.0, 4.0, 4.0], [-1.0, 1.0, 1.0]])
    assert ref.cosine_mask(s, 0.5).tolist() == [True, False, True]
    # the test is strict: cos == tau is not salient
    assert ref.cosine_mask(torch.tensor([[1.0, 1.0, 1.0]]), 1.0).tolist() == [False]


def test_saliency_stats_closed_form():
    g = torch.Generator().manual_seed(0)
    a, b = torch.randn(7, 33, generator=g), torch.randn(7, 33, generator=g)
    st = ref.saliency_stats(a, b)
    torch.testing.assert_close(st[:, 0], (a * b).sum(-1), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(st[:, 1], (a * a).sum(-1), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(st[:, 2], (b * b).sum(-1), rtol=1e-5, atol=1e-5)
    cos = ref.cosine_from_stats(st)
    torch.testing.assert_close(cos.float(), F.cosine_similarity(a, b, dim=-1), rtol=1e-5, atol=1e-6)


def _lens_case(seed, lens, H=4, Hkv=2, D=128):
    g = torch.Generator().manual_seed(seed)
    cu_q = np.concatenate([[0], np.cumsum([a for a, _ in lens])])
    cu_k = np.concatenate([[0], np.cumsum([b for _, b in lens])])
    q = torch.randn(int(cu_q[-1]), H, D, generator=g).to(BF)
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(BF)
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(BF)
    return q, k, v, cu_q, cu_k


def test_flash_attention_matches_sdpa():
    """Exact path equals torch's scaled_dot_product_attention per sequence (GQA expanded)."""
    q, k, v, cu_q, cu_k = _lens_case(1, [(5, 70), (64, 64), (1, 130)])
    out = ref.flash_attn_varlen(q, k, v, cu_q, cu_k, out_dtype=None, bf16_p=False)
    for b in range(3):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        qb = q[qs:qe].float().transpose(0, 1)
        kb = k[ks:ke].float().transpose(0, 1).repeat_interleave(2, 0)
        vb = v[ks:ke].float().transpose(0, 1).repeat_interleave(2, 0)
        want = F.scaled_dot_product_attention(qb, kb, vb).transpose(0, 1)
        torch.testing.assert_close(out[qs:qe], want, rtol=1e-4, atol=1e-5)
    # head h uses kv head h // 2: swapping kv heads changes the answer
    out2 = ref.flash_attn_varlen(q, k.flip(1), v.flip(1), cu_q, cu_k, out_dtype=None, bf16_p=False)
    assert (out2 - out).abs().max() > 1e-2


def test_blocked_bf16_softmax_close_to_exact_and_blockwise():
    q, k, v, cu_q, cu_k = _lens_case(2, [(16, 200)], H=2, Hkv=2)
    exact = ref.flash_attn_varlen(q, k, v, cu_q, cu_k, out_dtype=None, bf16_p=False)
    blocked = ref.flash_attn_varlen(q, k, v, cu_q, cu_k, out_dtype=None, bf16_p=True)
    rel = ((blocked - exact).abs().mean() / exact.abs().mean()).item()
    assert 0 < rel < 4e-3  # bf16 rounding of P is visible but small
    # the running-max blocking matters: rounding relative to the final max differs
    c2 = float(np.float32(np.float32(128 ** -0.5) * np.float32(ref.LOG2E)))
    qb, kb, vb = (t.float().transpose(0, 1) for t in (q, k, v))
    acc, l = ref._online_softmax_pv(qb, kb, vb, c2, 200)  # one block = final-max rounding
    assert not torch.equal((acc / l).transpose(0, 1), blocked)


def test_column_sparse_linearity_invariant():
    """C_old = attn(Q,K,V_old); dV = V_new - V_old on salient keys only; then
    C_old + softmax(QK^T/sqrt(D)) dV == attn(Q,K,V_new) for every row (the identity the
    reference's approximation rests on, attention.py:89-139)."""
    lens = [(40, 96), (20, 64)]
    q, k, v_old, cu_q, cu_k = _lens_case(3, lens, H=4, Hkv=4)
    g = torch.Generator().manual_seed(9)
    sal_k = np.array([3, 50, 95, 96 + 7, 96 + 33])
    v_new = v_old.clone()
    v_new[sal_k] = (v_old[sal_k].float() + torch.randn(len(sal_k), 4, 128, generator=g)).to(BF)
    dv = torch.zeros_like(v_old, dtype=torch.float32)
    dv[sal_k] = v_new[sal_k].float() - v_old[sal_k].float()
    c_old = ref.flash_attn_varlen(q, k, v_old, cu_q, cu_k, out_dtype=None, bf16_p=False)
    want = ref.flash_attn_varlen(q, k, v_new, cu_q, cu_k, out_dtype=None, bf16_p=False)
    o, stats, _ = ref.attention_sparse_varlen(q, k, dv, c_old, torch.zeros(0, 4, 128), cu_q, cu_k, [], 0.99)
    # o is bf16-rounded; the dV term carries the bf16 rounding of P
    assert (o.float() - want).abs().max().item() < 2e-2
    # stats are the closed form of the fp32 new rows vs C_old
    torch.testing.assert_close(ref.cosine_from_stats(stats).float(),
                               F.cosine_similarity(want.reshape(len(want), -1), c_old.reshape(len(want), -1), dim=-1),
                               rtol=1e-4, atol=1e-4)
    # dropping the dV term (or flipping its sign) breaks the identity
    o0, _, _ = ref.attention_sparse_varlen(q, k, torch.zeros_like(dv), c_old, torch.zeros(0, 4, 128), cu_q, cu_k,
                                           [], 0.99)
    assert (o0.float() - want).abs().max().item() > 5e-2


def test_column_sparse_salient_rows_take_o_sal():
    q, k, v, cu_q, cu_k = _lens_case(4, [(10, 40)], H=2, Hkv=2)
    c = ref.flash_attn_varlen(q, k, v, cu_q, cu_k)
    o_sal = torch.randn(2, 2, 128).to(BF)
    idx = [2, 7]
    o, st, m = ref.attention_sparse_varlen(q, k, torch.zeros_like(k), c, o_sal, cu_q, cu_k, idx, 0.99)
    assert torch.equal(o[idx], o_sal)
    # stats of salient rows come from bf16 o_sal vs C (attention_aux_kernels.cu:33-42)
    torch.testing.assert_close(st[idx], ref.saliency_stats(o_sal.float(), c[idx].float()))
    # unchanged rows: new == old -> cos == 1 -> not salient; random o_sal rows -> salient
    others = [i for i in range(10) if i not in idx]
    assert not m[others].any() and m[idx].all()


@pytest.mark.parametrize("seed", range(5))
def test_compaction_brute_force(seed):
    rng = np.random.default_rng(seed)
    T = int(rng.integers(0, 60))
    B = int(rng.integers(1, 5))
    mask = rng.random(T) < rng.random()
    cuts = np.sort(rng.integers(0, T + 1, size=B - 1))
    cu_q = np.concatenate([[0], cuts, [T]])
    cu_p = np.concatenate([[0], np.cumsum(rng.integers(0, 9, size=B))])
    idxs, cu = ref.compact(mask, cu_q)
    want = [t for t in range(T) if mask[t]]
    assert idxs.tolist() == want
    assert all(idxs[i] < idxs[i + 1] for i in range(len(idxs) - 1))
    assert cu.tolist() == [sum(1 for t in want if t < c) for c in cu_q]
    # per-sequence counts add up and every index lies in its sequence
    for b in range(B):
        for t in idxs[cu[b]:cu[b + 1]]:
            assert cu_q[b] <= t < cu_q[b + 1]
    # fused_offset: K-space row = Q-space index + prompt rows of all sequences up to and including its own
    k = ref.fused_offset(idxs, cu_p, cu)
    for j, t in enumerate(idxs):
        b = max(i for i in range(B) if cu[i] <= j < cu[i + 1]) if cu[-1] else 0
        assert k[j] == t + cu_p[b + 1]


def test_k_block_masks_brute_force():
    cu_k = [0, 100, 130]
    cu_s = [0, 3, 4]
    idx = [0, 63, 64, 129]
    m = ref.k_block_masks(idx, cu_s, cu_k, 100)
    assert m.shape == (2, 2)
    assert int(m[0, 0]) == (1 | (1 << 63)) and int(m[0, 1]) == 1 and int(m[1, 0]) == (1 << 29) and int(m[1, 1]) == 0


def test_cache_ops_round_trips():
    g = torch.Generator().manual_seed(5)
    cache = torch.randn(60, 8, generator=g)
    starts = torch.tensor([-1, 40, 2, -1, 17], dtype=torch.long)
    ids = torch.tensor([2, 4, 1])
    cu_k = [0, 10, 22, 30]
    cu_q = [0, 4, 10, 12]
    x = torch.randn(30, 8, generator=g)
    c2 = ref.reset_full(cache, x, starts, cu_k, ids)
    assert torch.equal(ref.get_seqs(c2, starts, cu_k, ids, 30), x)
    assert torch.equal(c2[2:12], x[0:10]) and torch.equal(c2[17:29], x[10:22]) and torch.equal(c2[40:48], x[22:30])
    xq = torch.randn(12, 8, generator=g)
    c3 = ref.reset_block(cache, xq, starts, cu_k, cu_q, ids)
    assert torch.equal(ref.get_block(c3, starts, cu_k, cu_q, ids, 12), xq)
    assert torch.equal(c3[2 + 6:12], xq[0:4])  # tail 4 rows of a 10-row sequence
    nv = torch.randn(2, 8, generator=g)
    c4 = ref.scatter_update(cache, nv, [9, 22], cu_k, starts, ids)
    assert torch.equal(c4[2 + 9], nv[0]) and torch.equal(c4[40], nv[1])
    assert torch.equal(ref.gather_rows_2D(cache, [3, 1]), cache[[3, 1]])


def test_swiglu_matches_per_row_loop():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(5, 16, generator=g).to(BF)
    wgu = (torch.randn(24, 16, generator=g) * 0.3).to(BF)
    wd = (torch.randn(16, 12, generator=g) * 0.3).to(BF)
    y = ref.swiglu_ffn(x, wgu, wd)
    for r in range(5):
        gate = ref.bf16_round(x[r].float() @ wgu[:12].float().t())
        up = ref.bf16_round(x[r].float() @ wgu[12:].float().t())
        h = ref.bf16_round(gate * torch.sigmoid(gate) * up)
        torch.testing.assert_close(y[r], h @ wd.float().t(), rtol=1e-5, atol=1e-5)
    # swapping the gate and up halves changes the result (silu is not symmetric)
    y2 = ref.swiglu_ffn(x, torch.cat([wgu[12:], wgu[:12]]), wd)
    assert (y2 - y).abs().max() > 1e-3


def test_moe_gate_and_experts_brute_force():
    g = torch.Generator().manual_seed(7)
    T, Hd, E, K, I = 6, 16, 8, 3, 4
    x = torch.randn(T, Hd, generator=g).to(BF)
    wr = torch.randn(E, Hd, generator=g).to(BF)
    w, ids = ref.moe_gate(x, wr, K)
    w1 = (torch.randn(E, 2 * I, Hd, generator=g) * 0.3).to(BF)
    w2 = (torch.randn(E, Hd, I, generator=g) * 0.3).to(BF)
    out = ref.naive_experts(x, w1, w2, w, ids)
    for t in range(T):
        logits = [float((x[t].float() * wr[e].float()).sum()) for e in range(E)]
        mx = max(logits)
        ex = [math.exp(l - mx) for l in logits]
        p = [a / sum(ex) for a in ex]
        top = sorted(range(E), key=lambda e: -p[e])[:K]
        assert ids[t].tolist() == top
        torch.testing.assert_close(w[t].float(), torch.tensor([p[e] for e in top]).to(BF).float())
        acc = torch.zeros(Hd)
        for kk, e in enumerate(top):
            gu = ref.bf16_round(x[t].float() @ w1[e].float().t())
            h = ref.bf16_round(F.silu(gu[:I]) * gu[I:])
            acc += ref.bf16_round((h @ w2[e].float().t()) * w[t, kk].float())
        torch.testing.assert_close(out[t], acc, rtol=1e-5, atol=1e-5)
    wn, _ = ref.moe_gate(x, wr, K, renormalize=True)
    torch.testing.assert_close(wn.float().sum(-1), torch.ones(T), rtol=1e-2, atol=1e-2)


def test_moe_align_invariants():
    rng = np.random.default_rng(8)
    ids = rng.integers(0, 5, size=(11, 3))
    sorted_ids, eids, npp = ref.moe_align_block_size(ids, 4, 5)
    S = ids.size
    assert npp % 4 == 0 and len(sorted_ids) == npp and len(eids) == npp // 4
    real = sorted_ids[sorted_ids < S]
    assert sorted(real.tolist()) == list(range(S))  # a permutation of all slots
    flat = ids.reshape(-1)
    for blk, e in enumerate(eids):
        for s in sorted_ids[4 * blk:4 * blk + 4]:
            if s < S:
                assert flat[s] == e  # each block is owned by one expert
    # stable: within an expert the slots keep their flattened order
    for e in range(5):
        own = [s for s in sorted_ids if s < S and flat[s] == e]
        assert own == sorted(own)


def test_synthetic_perturbation_known_answer():
    """Config-0 style: unperturbed rows keep cos == 1; rows perturbed with sigma = 0.5 x row
    RMS have cos ~ 1/sqrt(1.25) = 0.894 < 0.99, so the salient set is the perturbed set."""
    g = torch.Generator().manual_seed(10)
    old = torch.randn(64, 4096, generator=g)
    new = old.clone()
    pert = torch.tensor(sorted(torch.randperm(64, generator=g)[:7].tolist()))
    rms = old[pert].pow(2).mean(-1, keepdim=True).sqrt()
    new[pert] += 0.5 * rms * torch.randn(7, 4096, generator=g)
    st = ref.saliency_stats(new, old)
    mask = ref.cosine_mask(st, 0.99)
    assert torch.nonzero(mask).squeeze(-1).tolist() == pert.tolist()
    cos = ref.cosine_from_stats(st)[pert]
    assert ((cos - 1 / math.sqrt(1.25)).abs() < 0.02).all()


def test_rope_pinned_by_identity_norm_and_complex_form():
    """RoPE restatement: position 0 leaves x unchanged, each (d, d+64) pair keeps its length,
    and the rotation equals the complex product (x1 + i x2) e^{i p theta_d} with
    theta_d = base^(-2d/D) (a swapped sin sign or a half-swap fails all three)."""
    g = torch.Generator().manual_seed(3)
    cos, sin = ref.rope_tables(128, 4096, 10000.0)
    x = torch.randn(16, 4, 128, generator=g).to(BF)
    assert torch.equal(ref.rope_neox(x, cos, sin, torch.zeros(16, dtype=torch.long)), x)
    pos = torch.randint(0, 4096, (16,), generator=g)
    y = ref.rope_neox(x, cos, sin, pos).float()
    n_in = x.float()[..., :64] ** 2 + x.float()[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert torch.allclose(n_out, n_in, rtol=2e-2, atol=1e-3)
    theta = 10000.0 ** (-torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    z = torch.complex(x.double()[..., :64], x.double()[..., 64:]) * torch.exp(
        1j * pos.double()[:, None, None] * theta)
    want = torch.cat((z.real, z.imag), -1)
    assert (y.double() - want).abs().max() < 0.02 * want.abs().max()
    # positions past the table are clamped to its last row
    assert torch.equal(ref.rope_neox(x, cos, sin, torch.full((16,), 10 ** 6)),
                       ref.rope_neox(x, cos, sin, torch.full((16,), 4095)))


def test_rms_norm_unit_rms_and_weight():
    g = torch.Generator().manual_seed(4)
    x = (3.0 * torch.randn(32, 128, generator=g)).to(BF)
    one = torch.ones(128, dtype=BF)
    y = ref.rms_norm(x, one, 1e-6).float()
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(32), rtol=2e-2)
    w = torch.linspace(0.5, 2.0, 128).to(BF)
    assert torch.allclose(ref.rms_norm(x, w, 1e-6).float(), (y * w.float()), rtol=1e-2, atol=1e-2)


def test_salient_kv_project_per_row_loop():
    """Composition check: per-row loop of linear (+bias) -> k_norm -> RoPE vs the batched form."""
    g = torch.Generator().manual_seed(5)
    Hkv, hid = 2, 64
    hidden = torch.randn(10, hid, generator=g).to(BF)
    w = (0.1 * torch.randn(2 * Hkv * 128, hid, generator=g)).to(BF)
    b = (0.1 * torch.randn(2 * Hkv * 128, generator=g)).to(BF)
    kn = (1 + 0.1 * torch.randn(128, generator=g)).to(BF)
    pos = torch.arange(100, 110)
    cos, sin = ref.rope_tables(128, 512, 10000.0)
    idx = torch.tensor([7, 2, 5])
    k, v = ref.salient_kv_project(hidden, idx, w, b, pos, cos, sin, Hkv, kn, 1e-6)
    for j, r in enumerate(idx.tolist()):
        kv = (sum(hidden[r].float()[c] * w.float()[:, c] for c in range(hid)) + b.float()).to(BF)
        kr = kv[:Hkv * 128].view(Hkv, 128)
        assert torch.allclose(v[j].float(), kv[Hkv * 128:].view(Hkv, 128).float(), atol=1e-2)
        for h in range(Hkv):
            xf = kr[h].float()
            xn = ((xf / torch.sqrt(xf.pow(2).mean() + 1e-6)).to(BF).float() * kn.float()).to(BF).float()
            p = int(pos[r])
            c, s_ = cos[p], sin[p]
            want = torch.cat((xn[:64] * c - xn[64:] * s_, xn[64:] * c + xn[:64] * s_)).to(BF).float()
            assert (k[j, h].float() - want).abs().max() <= 0.05


def test_add_rms_norm_consistency_and_loop():
    """Fused residual form: a zero residual reduces to rms_norm; residual_out is the bf16 sum; y
    is normalised from the fp32 sum (not from the rounded residual), checked per row."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(6, 256, generator=g).to(BF)
    r = (2 * torch.randn(6, 256, generator=g)).to(BF)
    w = (1 + 0.1 * torch.randn(256, generator=g)).to(BF)
    y0, r0 = ref.add_rms_norm(x, torch.zeros_like(x), w, 1e-6)
    assert torch.equal(y0, ref.rms_norm(x, w, 1e-6)) and torch.equal(r0, x)
    y, ro = ref.add_rms_norm(x, r, w, 1e-6)
    for i in range(6):
        s = x[i].double() + r[i].double()
        assert torch.equal(ro[i], s.float().to(BF))
        n = (s / torch.sqrt((s * s).mean() + 1e-6)).float().to(BF).double() * w.double()
        assert (y[i].double() - n).abs().max() <= 2 ** -7 * n.abs().max()


# ---------------------------------------------------------------------------
# sparse_attention_step (attention.py:64-178), pinned end to end by what the mathematics fixes
# ---------------------------------------------------------------------------
def _dense_attn(q, k, v, cu_q, cu_k):
    """Exact fp32 softmax(QK^T/sqrt(D))V per sequence via torch SDPA (GQA expanded); the
    textbook operation the whole sparse step approximates."""
    Tq, H, D = q.shape
    g = H // k.shape[1]
    out = torch.zeros(Tq, H, D)
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        if qe == qs:
            continue
        qb = q[qs:qe].float().transpose(0, 1)
        kb = k[ks:ke].float().transpose(0, 1).repeat_interleave(g, 0)
        vb = v[ks:ke].float().transpose(0, 1).repeat_interleave(g, 0)
        out[qs:qe] = F.scaled_dot_product_attention(qb, kb, vb).transpose(0, 1)
    return out


def _step_case(seed, lens, q_pruned, n_sal_per_seq, H=4, Hkv=2, D=128, sigma=1.0):
    """Ragged batch: lens = [(prompt, response)]. Q-pruned: the queried rows are the
    responses; refresh: every row. The previous salient set is drawn per sequence from the
    response rows; its V rows get a fresh value (v_new)."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    cu_k = np.concatenate([[0], np.cumsum([p + r for p, r in lens])]).astype(np.int64)
    cu_p = np.concatenate([[0], np.cumsum([p for p, _ in lens])]).astype(np.int64)
    cu_q = (np.concatenate([[0], np.cumsum([r for _, r in lens])]) if q_pruned else cu_k).astype(np.int64)
    Tq, Tk = int(cu_q[-1]), int(cu_k[-1])
    q = torch.randn(Tq, H, D, generator=g).to(BF)
    k = torch.randn(Tk, Hkv, D, generator=g).to(BF)
    v_old = torch.randn(Tk, Hkv, D, generator=g).to(BF)
    sidx, kidx, cu_s = [], [], [0]
    for b, (p, r) in enumerate(lens):
        sel = np.sort(rng.choice(r, size=min(r, n_sal_per_seq[b]), replace=False))
        sidx += ((cu_q[b] + sel) if q_pruned else (cu_k[b] + p + sel)).tolist()
        kidx += (cu_k[b] + p + sel).tolist()
        cu_s.append(len(sidx))
    sidx, kidx, cu_s = (np.asarray(a, np.int64) for a in (sidx, kidx, cu_s))
    v_new = (v_old[kidx].float() + sigma * torch.randn(len(kidx), Hkv, D, generator=g)).to(BF)
    return dict(q=q, k=k, v_old=v_old, v_new=v_new, cu_q=cu_q, cu_k=cu_k, cu_p=cu_p, sidx=sidx, kidx=kidx,
                cu_s=cu_s, q_pruned=q_pruned)


def _run_step(c, c_old, tau=0.99):
    return ref.sparse_attention_step(c["q"], c["k"], c["v_new"], c["v_old"], c_old, c["cu_q"], c["cu_k"], c["cu_s"],
                                     c["sidx"], c["kidx"] if c["q_pruned"] else None, c["cu_p"], tau)


def _check_step(c, c_old, res, tau=0.99):
    """The properties a correct sparse step has, independent of how it is composed:
    (1) the V cache changes exactly at the salient K rows and holds v_new there;
    (2) every queried row's new context equals exact attn(Q, K, V_new) to bf16 rounding --
        salient rows because they are recomputed, the others by linearity of P.V;
    (3) the next salient set is {rows : cos(new, C_old) < tau} of those exact rows (outside
        the tau band), ascending, with cu_salientlens its per-sequence split;
    (4) Q-pruned: idx_salient_row_k is each index plus its sequence's prompt length
        (a per-row loop); refresh: it is None."""
    q, k, cu_q, cu_k = c["q"], c["k"], c["cu_q"], c["cu_k"]
    v_upd = c["v_old"].clone()
    v_upd[torch.as_tensor(c["kidx"])] = c["v_new"]
    assert torch.equal(res["v_cache"], v_upd), "V cache"
    changed = (res["v_cache"] != c["v_old"]).flatten(1).any(1).nonzero().squeeze(-1).numpy()
    assert set(changed.tolist()) <= set(c["kidx"].tolist())
    exact = _dense_attn(q, k, v_upd, cu_q, cu_k)
    sal = torch.as_tensor(c["sidx"])
    from tests._tol import assert_bf16_close
    # against the exact product the step carries two bf16 roundings (P before P.V and the
    # output) -> mean relative 3e-3 here; every composition mistake below moves rows by >10%
    assert_bf16_close(res["new_c"][sal], exact[sal], mean_rel=3e-3, what="salient rows")
    keep = torch.ones(len(q), dtype=torch.bool)
    keep[sal] = False
    assert_bf16_close(res["new_c"][keep], exact[keep], mean_rel=3e-3, what="non-salient rows")
    cos = F.cosine_similarity(exact.flatten(1).double(), c_old.float().flatten(1).double(), dim=-1).numpy()
    want = cos < tau
    band = np.abs(cos - tau) <= 1e-4  # fp32 paths vs the exact cosine: stay clear of the edge
    got = res["mask"].numpy()
    assert ((got == want) | band).all(), "salient set"
    idxs = res["idx_salient_row"]
    assert np.array_equal(idxs, np.nonzero(got)[0]) and np.all(np.diff(idxs) > 0)
    for b in range(len(cu_q) - 1):
        lo, hi = res["cu_salientlens"][b], res["cu_salientlens"][b + 1]
        assert np.all((idxs[lo:hi] >= cu_q[b]) & (idxs[lo:hi] < cu_q[b + 1]))
        assert hi - lo == got[cu_q[b]:cu_q[b + 1]].sum()
    if c["q_pruned"]:
        # the K-space row of each salient query row is the same token: same sequence, and the
        # same offset into its response (K rows of a sequence are prompt then response)
        got_k = np.asarray(res["idx_salient_row_k"])
        assert got_k.shape == idxs.shape
        for i, j in zip(idxs, got_k):
            b = int(np.searchsorted(cu_q, i, side="right")) - 1
            assert cu_k[b] <= j < cu_k[b + 1]
            plen = (cu_k[b + 1] - cu_k[b]) - (cu_q[b + 1] - cu_q[b])
            assert j - cu_k[b] - plen == i - cu_q[b]
    else:
        assert res["idx_salient_row_k"] is None


STEP_CASES = [
    ("qpruned_ragged", [(40, 96), (16, 48), (64, 130)], True, [9, 5, 20]),
    ("refresh_ragged", [(40, 96), (16, 48), (64, 130)], False, [9, 5, 20]),
    ("qpruned_empty_seq", [(32, 64), (8, 40)], True, [0, 6]),
    ("qpruned_no_salient", [(32, 64), (8, 40)], True, [0, 0]),
    ("refresh_all_salient", [(16, 24), (8, 16)], False, [24, 16]),
    ("qpruned_single_rows", [(20, 33), (5, 1)], True, [1, 1]),
]


@pytest.mark.parametrize("name,lens,q_pruned,nsal", STEP_CASES, ids=[s[0] for s in STEP_CASES])
def test_sparse_step_pinned_by_exact_attention(name, lens, q_pruned, nsal):
    c = _step_case(11, lens, q_pruned, nsal)
    # C_old: the exact fp32 context of the previous step (attn with the pre-update V)
    c_old = _dense_attn(c["q"], c["k"], c["v_old"], c["cu_q"], c["cu_k"])
    res = _run_step(c, c_old)
    _check_step(c, c_old, res)
    if nsal and sum(nsal):
        assert res["mask"].any()  # sigma = 1 on V rows moves the contexts past tau somewhere


def _step_mutant(c, c_old, kind, tau=0.99):
    """Plausible composition mistakes of attention.py:64-178, built from the oracle's own
    pieces: the pins above must reject each of them."""
    q, k = c["q"], c["k"]
    sidx = torch.as_tensor(c["sidx"])
    kidx = torch.as_tensor(c["kidx"] if c["q_pruned"] else c["sidx"])
    if kind == "dv_at_q_rows":  # Q-pruned: scatter dV at the Q-space indices
        kidx_dv = sidx
    else:
        kidx_dv = kidx
    v_cache = c["v_old"].clone()
    dv = ref.bf16_round(c["v_new"].float() - v_cache[kidx].float())
    v_cache[kidx] = c["v_new"]
    v_for_osal = c["v_old"] if kind == "o_sal_old_cache" else v_cache
    o_sal = ref.flash_attn_varlen(q[sidx], k, v_for_osal, c["cu_s"], c["cu_k"])
    vd = torch.zeros_like(k, dtype=torch.float32)
    vd[kidx_dv] = dv
    newc, stats, mask = ref.attention_sparse_varlen(q, k, vd.to(BF), c_old, o_sal, c["cu_q"], c["cu_k"], sidx, tau)
    idxs, cu_sal = ref.compact(mask.numpy(), c["cu_q"])
    if kind == "offset_own_prompt":  # fused offset with the sequence's start instead of its end
        seg = np.searchsorted(cu_sal[1:], np.arange(len(idxs)), side="right")
        idx_k = idxs + c["cu_p"][seg]
    else:
        idx_k = ref.fused_offset(idxs, c["cu_p"], cu_sal) if c["q_pruned"] else None
    return dict(new_c=newc, v_cache=v_cache, stats=stats, mask=mask, idx_salient_row=idxs, cu_salientlens=cu_sal,
                idx_salient_row_k=idx_k)


@pytest.mark.parametrize("kind", ["o_sal_old_cache", "dv_at_q_rows", "offset_own_prompt"])
def test_sparse_step_pins_reject_composition_mistakes(kind):
    c = _step_case(12, [(40, 96), (16, 48), (64, 130)], True, [9, 5, 20])
    c_old = _dense_attn(c["q"], c["k"], c["v_old"], c["cu_q"], c["cu_k"])
    _check_step(c, c_old, _step_mutant(c, c_old, "none"))  # the faithful composition passes
    with pytest.raises(AssertionError):
        _check_step(c, c_old, _step_mutant(c, c_old, kind))


def test_config0_known_answer_through_the_step():
    """Config 0 (B=1, 128 prompt + 384 response, 32 heads x 128, tau = 0.99) run through the
    whole Q-pruned step. Each response query is a scaled copy of its own key row, so its
    attention is one-hot on that row to within e^-30; the previous salient set holds 20% of the
    response rows, and the V rows of half of them (10% of the responses) move by
    sigma = 0.5 x row RMS while the rest keep their value. Known answer: the new salient set
    is exactly the perturbed rows (cos ~ 1/sqrt(1.25) = 0.894), and its K-space rows are those
    rows + 128."""
    P, R, H, D = 128, 384, 32, 128
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
    cu_q = np.array([0, R]); cu_k = np.array([0, P + R]); cu_p = np.array([0, P])
    c_old = ref.flash_attn_varlen(q, k, v_old, cu_q, cu_k)  # the bf16 context cache
    res = ref.sparse_attention_step(q, k, v_new, v_old, c_old, cu_q, cu_k, np.array([0, len(sal)]), sal, P + sal,
                                    cu_p, 0.99)
    assert res["idx_salient_row"].tolist() == pert.tolist()
    assert res["cu_salientlens"].tolist() == [0, len(pert)]
    assert res["idx_salient_row_k"].tolist() == (P + pert).tolist()
    cos = ref.cosine_from_stats(res["stats"]).numpy()
    assert np.all(np.abs(cos[pert] - 1 / math.sqrt(1.25)) < 0.03)
    assert np.all(np.delete(cos, pert) > 0.999)
