"""The benchmark configurations at their full sizes on the GPU.

Products (4a, 4b, 5.2, RoPE) are compared with the oracle over every output
element, bit for bit.  Contractions (1, 2, 3, 5.1, 5.3) are compared with the
oracle's exact per-output sum on a seeded sample of output positions (the
full single-threaded oracle would take minutes), and over every element with
size-independent checks: all finite, and within the same tolerance of a
float64 torch reference evaluated on the GPU."""
import numpy as np
import pytest
import torch

import oracle
from parity_util import check, ref64_gpu

pytestmark = pytest.mark.gpu


def _decay(t, gamma):
    i = torch.arange(t, dtype=torch.float64)
    d = i[:, None] - i[None, :]
    return torch.where(d >= 0, gamma ** d.clamp(min=0), torch.zeros(())).float()


def _rope(s, d):
    pos = torch.arange(s, dtype=torch.float64)[:, None]
    i = torch.arange(d, dtype=torch.float64)[None, :] % (d // 2)
    return torch.cos(pos * 10000.0 ** (-2.0 * i / d)).to(torch.float16)


def _contraction(eq, a, b, rtol, samples=4096):
    from pto_einsum import einsum

    print(f"config {eq} {tuple(a.shape)} x {tuple(b.shape)} {a.dtype}", flush=True)
    ga, gb = a.cuda(), b.cuda()
    got = einsum(eq, ga, gb)
    assert bool(torch.isfinite(got).all())
    # Every element against a float64 GPU reference of the same (up-cast) inputs.
    ref64 = ref64_gpu(eq, ga, gb)
    scale = float(ref64.abs().max())
    err = float((got.double() - ref64).abs().max())
    assert err <= rtol * scale, f"{eq}: max err {err:.3e} > {rtol * scale:.3e}"
    del ref64
    # Sampled positions against the oracle's exact per-output sums.
    idx = np.random.default_rng(0).integers(0, got.numel(), samples)
    want = oracle.sampled(eq, a.float().numpy(), b.float().numpy(), idx)
    check(got.flatten()[torch.from_numpy(idx).cuda()].cpu().numpy(), want, False, rtol, eq)


def test_config1():
    g = torch.Generator().manual_seed(1)
    a, b = torch.rand(256, 256, generator=g), torch.rand(256, 256, generator=g)
    from pto_einsum import einsum

    got = einsum("ij,jk->ik", a.cuda(), b.cuda()).cpu().numpy()
    check(got, oracle.einsum("ij,jk->ik", a.numpy(), b.numpy()), False, 1e-4, "config 1")


def test_config2():
    g = torch.Generator().manual_seed(2)
    _contraction("bji,bjk->bik", torch.randn(16, 777, 1000, generator=g), torch.randn(16, 777, 1536, generator=g), 1e-4)


def test_config3():
    g = torch.Generator().manual_seed(3)
    s = 128 ** -0.5
    a = (torch.randn(4, 2048, 32, 128, generator=g) * s).half()
    b = (torch.randn(4, 2048, 32, 128, generator=g) * s).half()
    _contraction("bshd,bthd->bsht", a, b, 2e-3)


def test_config4a_hadamard_decay_mask():
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(4)
    x, m = torch.rand(8192, 8192, generator=g), _decay(8192, 0.99)
    got = einsum("ts,ts->ts", x.cuda(), m.cuda()).cpu().numpy()
    want = oracle.hadamard(x.numpy(), m.numpy())
    assert np.count_nonzero((want != 0) & (np.abs(want) < 1.17549435e-38)) > 0  # subnormals present
    check(got, want, True, 0, "config 4a")


def test_config4b_rmsnorm_broadcast():
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(5)
    a = torch.randn(8, 4096, 4096, generator=g).half()
    w = (torch.rand(4096, generator=g) + 0.5).half()
    got = einsum("bsd,d->bsd", a.cuda(), w.cuda()).cpu().numpy()
    check(got, oracle.einsum("bsd,d->bsd", a.float().numpy(), w.float().numpy()), True, 0, "config 4b")


def test_config5_linear_attention_chain():
    """tn,sn->ts (fp16 -> fp32), ts,ts->ts with the causal decay mask (fp32),
    ts,sp->tp (fp32 intermediate x V up-cast to fp32)."""
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(6)
    s = 128 ** -0.5
    q = (torch.randn(4096, 128, generator=g) * s).half()
    k = (torch.randn(4096, 128, generator=g) * s).half()
    v = torch.randn(4096, 128, generator=g).half().float()
    mask = _decay(4096, 0.995)
    _contraction("tn,sn->ts", q, k, 2e-3)
    a1 = einsum("tn,sn->ts", q.cuda(), k.cuda())
    a2 = einsum("ts,ts->ts", a1, mask.cuda())
    check(a2.cpu().numpy(), oracle.hadamard(a1.cpu().numpy(), mask.numpy()), True, 0, "5.2")
    _contraction("ts,sp->tp", a2.cpu(), v, 1e-4)


def test_config5_rope_broadcast():
    from pto_einsum import einsum

    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 4096, 32, 128, generator=g).half()
    c = _rope(4096, 128)
    got = einsum("bshd,sd->bshd", x.cuda(), c.cuda()).cpu().numpy()
    check(got, oracle.einsum("bshd,sd->bshd", x.float().numpy(), c.float().numpy()), True, 0, "5.R")


@pytest.mark.parametrize("s0,s1", [((4096, 1024), (1024, 4096)),      # 256x128 tiles in whole rounds
                                   ((2000, 777), (777, 4100)),        # 128x128, partial, K tail
                                   ((4000, 300), (300, 2200))])       # 128x128, partial in M and N
def test_large_fp32_gemm_tilings(s0, s1):
    """Large float32 GEMMs through the automatic tile choice (every tile
    shape is also forced directly in test_gpu_components)."""
    g = torch.Generator().manual_seed(8)
    _contraction("ij,jk->ik", torch.randn(s0, generator=g), torch.randn(s1, generator=g), 1e-4, samples=2048)
