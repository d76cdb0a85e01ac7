"""GPU parity of the salient-row K/V projection (the step before the sparse attention,
llada.py:103-146): the gathered linear (dyllm_linear) and the k_norm + RoPE + K-cache scatter +
V split epilogue (dyllm_kv_rope_scatter), against the CPU oracle on seeded inputs.

The epilogue is compared bit-exactly when the kernel gets the same bf16 kv rows and the same
cos / sin tables as the oracle (no k_norm; with k_norm the fp32 mean's summation order may move
a value by one bf16 ulp, so that case uses the bf16 tolerance). Cache rows that no salient row
maps to must stay untouched. The linear is compared within the bf16 tolerance (max abs 2e-2,
mean rel 1e-3)."""
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _ops():
    from dyllm_amd import ops

    return ops


def _case(seed, lens_k, lens_q, seq_ids, hkv, n_sal_per_seq):
    """Packed K-space rows (cu_k), Q-pruned queried rows (the tail lens_q of each sequence) and
    a salient subset of them; a K cache slab whose sequences start at scattered rows."""
    g = torch.Generator().manual_seed(seed)
    B = len(lens_k)
    cu_k = [0]
    cu_q = [0]
    for lk, lq in zip(lens_k, lens_q):
        cu_k.append(cu_k[-1] + lk)
        cu_q.append(cu_q[-1] + lq)
    starts = torch.zeros(max(seq_ids) + 1, dtype=torch.long)
    pos = 3
    for b, sid in enumerate(seq_ids):
        starts[sid] = pos
        pos += lens_k[b] + 5
    cache_rows = pos + 2
    idx_q, idx_k = [], []
    for b in range(B):
        sel = torch.randperm(lens_q[b], generator=g)[: n_sal_per_seq[b]].sort().values
        for t in sel.tolist():
            idx_q.append(cu_q[b] + t)
            idx_k.append(cu_k[b] + (lens_k[b] - lens_q[b]) + t)
    return dict(g=g, B=B, cu_k=torch.tensor(cu_k, dtype=torch.int32), cu_q=torch.tensor(cu_q, dtype=torch.int32),
                seq_ids=torch.tensor(seq_ids, dtype=torch.long), starts=starts, cache_rows=cache_rows,
                idx_q=torch.tensor(idx_q, dtype=torch.long), idx_k=torch.tensor(idx_k, dtype=torch.long), hkv=hkv)


def _dest_rows(c):
    cu = c["cu_k"].tolist()
    out = []
    for k in c["idx_k"].tolist():
        b = max(i for i in range(c["B"]) if cu[i] <= k)
        out.append(int(c["starts"][c["seq_ids"][b]]) + (k - cu[b]))
    return torch.tensor(out, dtype=torch.long)


@pytest.mark.parametrize("k_norm", [False, True])
def test_kv_rope_scatter_matches_oracle(dev, k_norm):
    ops = _ops()
    c = _case(11, [37, 300, 64], [20, 256, 64], [5, 0, 3], hkv=4, n_sal_per_seq=[3, 40, 64])
    print(f"[kv_rope] k_norm={k_norm} n={len(c['idx_q'])}", flush=True)
    g = c["g"]
    n, hkv = len(c["idx_q"]), c["hkv"]
    kvs = hkv * 128
    Tq = int(c["cu_q"][-1])
    kv = (torch.randn(n, 2 * kvs, generator=g) * 2.0).to(BF)
    positions = torch.randint(0, 9000, (Tq,), generator=g)        # some past the 8192-row table
    cos, sin = ref.rope_tables(128, 8192, 10000.0)
    kn = (1 + 0.2 * torch.randn(128, generator=g)).to(BF) if k_norm else None
    cache0 = torch.randn(c["cache_rows"], kvs, generator=g).to(BF)

    k_cache = cache0.to(dev)
    v = ops.kv_rope_scatter(kv.to(dev), hkv, positions.to(dev), cos.to(dev), sin.to(dev), k_cache,
                            c["idx_k"].to(dev), c["cu_k"].to(dev), c["starts"].to(dev), c["seq_ids"].to(dev),
                            pos_idx=c["idx_q"].to(dev), k_norm_weight=None if kn is None else kn.to(dev), eps=1e-6)
    torch.cuda.synchronize()

    k = kv[:, :kvs].view(n, hkv, 128)
    if kn is not None:
        k = ref.rms_norm(k, kn, 1e-6)
    k_want = ref.rope_neox(k, cos, sin, positions[c["idx_q"]]).view(n, kvs)
    want = cache0.clone()
    dest = _dest_rows(c)
    want[dest] = k_want
    got = k_cache.cpu()
    assert torch.equal(v.cpu().view(n, kvs), kv[:, kvs:]), "v rows must be copied unchanged"
    untouched = torch.ones(c["cache_rows"], dtype=torch.bool)
    untouched[dest] = False
    assert torch.equal(got[untouched], cache0[untouched]), "cache rows of non-salient keys changed"
    if kn is None:
        assert torch.equal(got[dest], k_want)
    else:
        assert_bf16_close(got[dest], k_want, what="k_norm + rope")


def test_kv_rope_scatter_device_count(dev):
    """With rows_dev only the first count rows are processed; later cache rows stay untouched."""
    ops = _ops()
    c = _case(12, [128, 96], [128, 96], [1, 0], hkv=2, n_sal_per_seq=[30, 20])
    g = c["g"]
    n, hkv = len(c["idx_q"]), c["hkv"]
    kvs = hkv * 128
    kv = torch.randn(n, 2 * kvs, generator=g).to(BF)
    positions = torch.arange(int(c["cu_q"][-1]), dtype=torch.long)
    cos, sin = ref.rope_tables(128, 4096, 500000.0)
    cache0 = torch.randn(c["cache_rows"], kvs, generator=g).to(BF)
    k_cache = cache0.to(dev)
    cnt = torch.tensor([17], dtype=torch.int32, device=dev)
    v = ops.kv_rope_scatter(kv.to(dev), hkv, positions.to(dev), cos.to(dev), sin.to(dev), k_cache,
                            c["idx_k"].to(dev), c["cu_k"].to(dev), c["starts"].to(dev), c["seq_ids"].to(dev),
                            pos_idx=c["idx_q"].to(dev), count=cnt)
    torch.cuda.synchronize()
    dest = _dest_rows(c)
    k_want = ref.rope_neox(kv[:17, :kvs].view(17, hkv, 128), cos, sin, positions[c["idx_q"][:17]]).view(17, kvs)
    got = k_cache.cpu()
    assert torch.equal(got[dest[:17]], k_want)
    assert torch.equal(got[dest[17:]], cache0[dest[17:]])
    assert torch.equal(v.cpu()[:17].view(17, kvs), kv[:17, kvs:])


# (200, 3584, 512): 14 output-column tiles, a tile count below the CU count and not a multiple of 8
@pytest.mark.parametrize("rows,n_out,k_in,bias", [(920, 8192, 4096, False), (37, 1024, 3584, True),
                                                  (300, 4096, 12288, False), (1, 264, 128, True),
                                                  (200, 3584, 512, True)])
def test_linear_gathered_matches_oracle(dev, rows, n_out, k_in, bias):
    ops = _ops()
    print(f"[linear] rows={rows} n={n_out} k={k_in} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(rows + n_out)
    T = rows + 50
    x = torch.randn(T, k_in, generator=g).to(BF)
    # outputs of std 0.5: the bf16 bound (max abs 2e-2) is one ulp up to magnitude 4
    w = (torch.randn(n_out, k_in, generator=g) * (0.5 / k_in ** 0.5)).to(BF)
    b = (torch.randn(n_out, generator=g) * 0.5).to(BF) if bias else None
    idx = torch.randperm(T, generator=g)[:rows].to(torch.int32)
    got = ops.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), rows_idx=idx.to(dev))
    torch.cuda.synchronize()
    want = x[idx.long()].float() @ w.float().t()
    if b is not None:
        want = want + b.float()
    assert_bf16_close(got.cpu(), want.to(BF), what="gathered linear")


def test_linear_device_count_leaves_tail(dev):
    ops = _ops()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(400, 512, generator=g).to(BF)
    w = (torch.randn(2048, 512, generator=g) * 0.05).to(BF)
    idx = torch.arange(399, -1, -1, dtype=torch.int32)
    cnt = torch.tensor([123], dtype=torch.int32, device=dev)
    got = ops.linear(x.to(dev), w.to(dev), rows_idx=idx.to(dev), count=cnt, hint=123)
    torch.cuda.synchronize()
    want = (x[idx.long()[:123]].float() @ w.float().t()).to(BF)
    assert_bf16_close(got[:123].cpu(), want, what="linear, device count")


def test_salient_kv_projection_end_to_end(dev):
    """dyllm_linear + dyllm_kv_rope_scatter against oracle.salient_kv_project (Dream-like GQA
    with bias, LLaDA-MoE-like k_norm)."""
    ops = _ops()
    for hkv, hid, bias, kn in ((4, 3584, True, False), (16, 2048, False, True)):
        c = _case(13 + hkv, [200, 150], [160, 150], [0, 1], hkv=hkv, n_sal_per_seq=[25, 31])
        g = c["g"]
        Tq = int(c["cu_q"][-1])
        hidden = torch.randn(Tq, hid, generator=g).to(BF)
        w = (torch.randn(2 * hkv * 128, hid, generator=g) * 0.02).to(BF)
        b = (torch.randn(2 * hkv * 128, generator=g) * 0.1).to(BF) if bias else None
        knw = (1 + 0.1 * torch.randn(128, generator=g)).to(BF) if kn else None
        positions = torch.randint(0, 4096, (Tq,), generator=g)
        cos, sin = ref.rope_tables(128, 4096, 10000.0)
        cache0 = torch.zeros(c["cache_rows"], hkv * 128, dtype=BF)
        k_cache = cache0.to(dev)
        kv = ops.linear(hidden.to(dev), w.to(dev), None if b is None else b.to(dev), rows_idx=c["idx_q"].to(dev))
        v = ops.kv_rope_scatter(kv, hkv, positions.to(dev), cos.to(dev), sin.to(dev), k_cache, c["idx_k"].to(dev),
                                c["cu_k"].to(dev), c["starts"].to(dev), c["seq_ids"].to(dev),
                                pos_idx=c["idx_q"].to(dev), k_norm_weight=None if knw is None else knw.to(dev))
        torch.cuda.synchronize()
        k_want, v_want = ref.salient_kv_project(hidden, c["idx_q"], w, b, positions, cos, sin, hkv, knw, 1e-6)
        assert_bf16_close(v.cpu(), v_want, what=f"v (hkv={hkv})")
        assert_bf16_close(k_cache.cpu()[_dest_rows(c)].view(-1, hkv, 128), k_want, what=f"k (hkv={hkv})")


@pytest.mark.parametrize("norm", [False, True])
def test_rope_in_place_matches_oracle(dev, norm):
    """dyllm_rope on the queries: every row rotated in place at its own position (with q_norm
    first when given); bit-exact without the norm."""
    ops = _ops()
    g = torch.Generator().manual_seed(21)
    rows, H = 333, 12
    x = (torch.randn(rows, H * 128, generator=g) * 1.5).to(BF)
    pos = torch.randint(0, 5000, (rows,), generator=g)
    cos, sin = ref.rope_tables(128, 4096, 10000.0)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(BF) if norm else None
    xd = x.to(dev)
    ops.rope_(xd, H, pos.to(dev), cos.to(dev), sin.to(dev), None if w is None else w.to(dev), 1e-6)
    torch.cuda.synchronize()
    xin = x.view(rows, H, 128)
    if w is not None:
        xin = ref.rms_norm(xin, w, 1e-6)
    want = ref.rope_neox(xin, cos, sin, pos).view(rows, H * 128)
    if w is None:
        assert torch.equal(xd.cpu(), want)
    else:
        assert_bf16_close(xd.cpu(), want, what="q_norm + rope")
