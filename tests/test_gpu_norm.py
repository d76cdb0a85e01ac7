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
