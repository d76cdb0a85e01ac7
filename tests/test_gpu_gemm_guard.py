"""GPU checks of two details of the gathered GEMM (csrc/gemm.hip) through the C ABI:

* negative gather ids are padding: the A row is not read (row 0 stands in) and the output row is
  not written, in the direct epilogue and in the split-K reduction (gemm_tile_rows, the store
  epilogue and gemm_partial_reduce_kernel); every other row equals the fp32 oracle within the bf16
  bound (max abs 2e-2, mean rel 1e-3);
* the SwiGLU epilogue's SiLU (hardware reciprocal instead of an IEEE division) stays within one
  bf16 ulp of bf16(g / (1 + exp(-g))) in fp32 over a sweep of g across the tails and around 0
  (activations.py:11-14 computes silu(g) * u in fp32 and rounds once), and the standalone
  dyllm_silu_and_mul gives the same bits on the same g and u."""
import numpy as np
import pytest
import torch

from tests._tol import assert_bf16_close

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("M,N,K", [(40, 256, 512), (300, 1024, 12288)])
def test_negative_gather_ids_are_padding(dev, M, N, K):
    from dyllm_amd import _lib, ops

    print(f"[gemm guard] M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M)
    src_rows = 2 * M
    x = torch.randn(src_rows, K, generator=g).to(BF)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(BF)
    ids = torch.randint(0, src_rows, (M,), generator=g, dtype=torch.int32)
    neg = torch.arange(M) % 7 == 3
    ids[neg] = -1 - torch.arange(int(neg.sum()), dtype=torch.int32)   # -1, -2, ...
    sentinel = torch.full((M, N), 7.0).to(BF)
    out = sentinel.to(dev)
    xd, wd, idd = x.to(dev), w.to(dev), ids.to(dev)
    lib = _lib.load()
    ws_bytes = lib.dyllm_linear_workspace_bytes(M, 0, N, K)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("dyllm_linear", xd.data_ptr(), xd.stride(0), idd.data_ptr(), M, None, 0, wd.data_ptr(), N, K, None,
              out.data_ptr(), ws.data_ptr(), ws_bytes, ops._stream())
    got = out.cpu()
    assert torch.equal(got[neg], sentinel[neg]), "a padding row was written"
    keep = ~neg
    want = (x[ids[keep].long()].float() @ w.float().t()).to(BF)
    assert_bf16_close(got[keep], want, what="gathered GEMM rows")


def test_swiglu_silu_within_one_ulp(dev):
    from dyllm_amd import ops

    hidden, inter = 256, 512
    M = hidden
    # bf16 gate values: the tails (|g| up to 90, where exp(-g) over/underflows) and a dense
    # neighbourhood of 0, M * inter of them
    rng = np.random.default_rng(0)
    vals = np.concatenate([np.linspace(-90, 90, 40_000), np.linspace(-4, 4, 60_000), rng.normal(0, 3, 31_072)])
    g = torch.from_numpy(vals[: M * inter].astype(np.float32)).to(BF).view(inter, M)
    # A row m = e_m, so gate[m, n] = w_gate[n, m] and up[m, n] = w_up[n, m] = 1 exactly
    w = torch.cat([g, torch.ones(inter, M, dtype=BF)], dim=0).contiguous()
    x = torch.eye(M, dtype=torch.float32).to(BF)
    h = ops.ffn_gate_up(x.to(dev), w.to(dev)).cpu().float()
    gf = g.t().float()
    want = (gf / (1.0 + torch.exp(-gf))).to(BF).float()
    # one bf16 ulp of the reference value (2^(e - 7) for |v| in [2^e, 2^(e+1)))
    ulp = torch.ldexp(torch.ones_like(want), torch.frexp(want.abs().clamp_min(2.0 ** -126))[1] - 8)
    diff = (h - want).abs()
    bad = diff > ulp
    assert not bad.any(), f"{int(bad.sum())} values differ by more than one bf16 ulp, e.g. g={gf[bad][:5].tolist()}"
    # the standalone SiLU-and-mul (dyllm_silu_and_mul, after a library gate_up GEMM) on the same g
    # and u: bit-identical to the fused epilogue, with u != 1 as well
    gu = torch.cat([g.t(), torch.ones(M, inter, dtype=BF)], dim=1).contiguous().to(dev)
    assert torch.equal(ops.silu_and_mul(gu).cpu().float(), h)
    u = (torch.randn(M, inter, generator=torch.Generator().manual_seed(3)) * 2).to(BF)
    h2 = ops.silu_and_mul(torch.cat([g.t(), u], dim=1).contiguous().to(dev)).cpu().float()
    want2 = (gf / (1.0 + torch.exp(-gf)) * u.float()).to(BF).float()
    ulp2 = torch.ldexp(torch.ones_like(want2), torch.frexp(want2.abs().clamp_min(2.0 ** -126))[1] - 8)
    bad2 = (h2 - want2).abs() > ulp2
    assert not bad2.any(), f"silu_and_mul: {int(bad2.sum())} values off by more than one bf16 ulp"


def test_silu_and_mul_strided_rows(dev):
    """dyllm_silu_and_mul through the C ABI on padded row strides (ld_in > 2I, ld_out > I) and an
    odd row count: every output element equals bf16(silu(g) * u) within one bf16 ulp of the fp32
    reference, and the padding columns of the output rows are left untouched."""
    from dyllm_amd import _lib, ops

    rows, inter, pad_in, pad_out = 37, 136, 16, 24
    g = torch.Generator().manual_seed(11)
    gu = (torch.randn(rows, 2 * inter + pad_in, generator=g) * 3).to(BF)
    sentinel = torch.full((rows, inter + pad_out), 5.0).to(BF)
    out = sentinel.to(dev)
    gud = gu.to(dev)
    _lib.call("dyllm_silu_and_mul", gud.data_ptr(), gu.shape[1], rows, inter, out.data_ptr(), out.shape[1], ops._stream())
    got = out.cpu()
    assert torch.equal(got[:, inter:], sentinel[:, inter:]), "padding columns were written"
    gf, uf = gu[:, :inter].float(), gu[:, inter:2 * inter].float()
    want = (gf / (1.0 + torch.exp(-gf)) * uf).to(BF).float()
    ulp = torch.ldexp(torch.ones_like(want), torch.frexp(want.abs().clamp_min(2.0 ** -126))[1] - 8)
    bad = (got[:, :inter].float() - want).abs() > ulp
    assert not bad.any(), f"{int(bad.sum())} values off by more than one bf16 ulp"
