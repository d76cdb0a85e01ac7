"""GPU parity of the decoder-layer RMSNorm (dyllm_rms_norm, layernorm.py:15-37) against the CPU
oracle: residual_out bit-exact (bf16 of the fp32 sum), y within the bf16 bound (the sum of
squares is reduced in another order than torch's mean, which can move a value by one ulp);
in-place use; the three model families' hidden sizes."""
import pytest
import torch

from oracle import dyllm_oracle as ref
from tests._tol import assert_bf16_close

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


@pytest.mark.parametrize("hidden", [4096, 3584, 2048, 8192, 1032])
def test_add_rms_norm_matches_oracle(dev, hidden):
    from dyllm_amd import ops

    print(f"[rms_norm] hidden={hidden}", flush=True)
    g = torch.Generator().manual_seed(hidden)
    rows = 300
    x = (3 * torch.randn(rows, hidden, generator=g)).to(BF)
    r = torch.randn(rows, hidden, generator=g).to(BF)
    w = (1 + 0.2 * torch.randn(hidden, generator=g)).to(BF)
    y, ro = ops.rms_norm(x.to(dev), w.to(dev), 1e-5, residual=r.to(dev))
    y_plain = ops.rms_norm(x.to(dev), w.to(dev), 1e-5)
    torch.cuda.synchronize()
    y_want, ro_want = ref.add_rms_norm(x, r, w, 1e-5)
    assert torch.equal(ro.cpu(), ro_want)
    assert_bf16_close(y.cpu(), y_want, what="add + rms_norm")
    assert_bf16_close(y_plain.cpu(), ref.rms_norm(x, w, 1e-5), what="rms_norm")


def test_rms_norm_in_place(dev):
    from dyllm_amd import ops

    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 4096, generator=g).to(BF)
    r = torch.randn(64, 4096, generator=g).to(BF)
    w = torch.ones(4096, dtype=BF)
    xd, rd = x.to(dev), r.to(dev)
    ops.rms_norm(xd, w.to(dev), 1e-6, residual=rd, out=xd, residual_out=rd)
    torch.cuda.synchronize()
    y_want, ro_want = ref.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(rd.cpu(), ro_want)
    assert_bf16_close(xd.cpu(), y_want, what="in place")


@pytest.mark.parametrize("refresh", [False, True])
def test_rms_norm_reads_cache_rows_in_place(dev, refresh):
    """x read straight from a row cache through the tail-block addressing (ops.CacheRows): the
    same bits as the norm of the packed copy (dyllm_get_block / get_seqs), for a ragged batch whose
    sequences sit in the slab out of batch order."""
    from dyllm_amd import ops

    print(f"[rms_norm] cache rows refresh={refresh}", flush=True)
    g = torch.Generator().manual_seed(3)
    hidden = 4096
    lens_k, lens_q = [300, 41, 129], [200, 41, 1]
    if refresh:
        lens_q = lens_k
    seq_ids = [5, 0, 2]
    starts = torch.full((8,), -1, dtype=torch.long)
    pos = 7
    for sid, L in zip([2, 5, 0], [lens_k[2], lens_k[0], lens_k[1]]):     # slab order differs from batch order
        starts[sid] = pos
        pos += L + 3
    slab = (2 * torch.randn(pos + 5, hidden, generator=g)).to(BF)
    cu_k = torch.tensor([0, 300, 341, 470], dtype=torch.int32)
    cu_q = torch.tensor([0] + list(torch.tensor(lens_q).cumsum(0).tolist()), dtype=torch.int32)
    T = int(cu_q[-1])
    r = torch.randn(T, hidden, generator=g).to(BF)
    w = (1 + 0.2 * torch.randn(hidden, generator=g)).to(BF)
    sd, std, sid, ckd, cqd = (t.to(dev) for t in (slab, starts, torch.tensor(seq_ids), cu_k, cu_q))
    rows = ops.CacheRows(sd, std, sid, ckd, cqd, T)
    packed = rows.materialize()
    want_p = ref.get_block(slab, starts, cu_k, cu_q, seq_ids, T)
    assert torch.equal(packed.cpu(), want_p)
    y, ro = ops.rms_norm(rows, w.to(dev), 1e-5, residual=r.to(dev))
    y2, ro2 = ops.rms_norm(packed, w.to(dev), 1e-5, residual=r.to(dev))
    y3 = ops.rms_norm(rows, w.to(dev), 1e-5)
    y4 = ops.rms_norm(packed, w.to(dev), 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y2.cpu()) and torch.equal(ro.cpu(), ro2.cpu()) and torch.equal(y3.cpu(), y4.cpu())
