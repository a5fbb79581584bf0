"""Fused linear-attention chain on the GPU against the oracle's three-step
chain (float32 intermediates).  The reference covers the chain with
tests/test_llm_ops.py:81-107 (T = S in {96, 320}, N = 64, P = 128, a
lower-triangular ones mask, both dtypes); these cases add benchmark config 5's
full size with its decay mask, partial tiles in every axis, several s splits,
float16 masks and values, dense masks and strided rows."""
import numpy as np
import pytest
import torch

import oracle
from parity_util import check

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-4, torch.float16: 2e-3}


def _decay(t, gamma):
    i = torch.arange(t, dtype=torch.float64)
    d = i[:, None] - i[None, :]
    return torch.where(d >= 0, gamma ** d.clamp(min=0), torch.zeros(())).float()


def _run(q, k, v, m, **kw):
    from pto_einsum import linear_attention

    print(f"linear_attention q{tuple(q.shape)} {q.dtype} v{tuple(v.shape)} {v.dtype} m {m.dtype} {kw}", flush=True)
    return linear_attention(q.cuda(), k.cuda(), v.cuda(), m.cuda(), **kw).cpu()


def _want(q, k, v, m):
    return oracle.linear_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), m.float().numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("T,S,N,P", [(96, 96, 64, 128), (320, 320, 64, 128)])
def test_reference_chain_cases(dtype, T, S, N, P):
    """The reference test's shapes and mask (torch.rand operands, tril ones)."""
    g = torch.Generator().manual_seed(T)
    q, k, v = (torch.rand(sh, generator=g).to(dtype) for sh in ((T, N), (S, N), (S, P)))
    m = torch.tril(torch.ones(T, S)).to(dtype)
    got = _run(q, k, v, m)
    check(got.numpy(), _want(q, k, v, m), False, RTOL[dtype], "linear_attention")
    # and the reference's own acceptance check against torch's 4-way einsum
    ref = torch.einsum("tn,sn,sp,ts->tp", q.double(), k.double(), v.double(), m.double())
    torch.testing.assert_close(got.double(), ref, rtol=1e-3, atol=1e-3 * float(ref.abs().max()))


@pytest.mark.parametrize("T,S,N,P,qk,vd,md", [
    (77, 130, 40, 200, torch.float16, torch.float32, torch.float32),   # partial t, s, p; N tail
    (130, 77, 128, 96, torch.float16, torch.float16, torch.float16),   # float16 values and mask
    (200, 333, 200, 64, torch.float16, torch.float32, torch.float32),  # N up to 256 (16 MFMA steps)
    (64, 256, 100, 130, torch.float32, torch.float32, torch.float32),  # float32 q/k, N not a step multiple
    (33, 65, 7, 5, torch.float32, torch.float16, torch.float32),       # tiny, odd everything
    (1, 1, 1, 1, torch.float16, torch.float16, torch.float16),
])
@pytest.mark.parametrize("dense", [False, True], ids=["causal", "dense"])
@pytest.mark.parametrize("precise", [False, True], ids=["split_pv", "f32_pv"])
def test_shapes_and_dtypes(T, S, N, P, qk, vd, md, dense, precise):
    g = torch.Generator().manual_seed(T * 7 + S)
    q = (torch.randn(T, N, generator=g) * N ** -0.5).to(qk)
    k = (torch.randn(S, N, generator=g) * N ** -0.5).to(qk)
    v = torch.randn(S, P, generator=g).to(vd)
    m = (torch.rand(T, S, generator=g) if dense else _decay(max(T, S), 0.97)[:T, :S]).to(md)
    got = _run(q, k, v, m, precise=precise)
    check(got.numpy(), _want(q, k, v, m), False, RTOL[qk], "linear_attention")


@pytest.mark.parametrize("vd", [torch.float16, torch.float32], ids=["v16", "v32"])
def test_split_pv_error_bound(vd):
    """The default P.V (bfloat16 terms at float32 accuracy) against float32
    MFMAs on the same inputs, and both against a float64 evaluation: the
    split leaves out at most 2^-22 |P||V| per product, so its error is that
    of float32 arithmetic -- bounded here by 2^-20 sum_s |P||V| per output
    (float32 accumulation over 2048 terms included), with a mean no larger
    than 1.25 times the float32 MFMAs' own."""
    g = torch.Generator().manual_seed(50)
    T, S, N, P = 512, 2048, 128, 128
    q = (torch.randn(T, N, generator=g) * N ** -0.5).half()
    k = (torch.randn(S, N, generator=g) * N ** -0.5).half()
    v = (torch.randn(S, P, generator=g) * 3).to(vd)
    m = _decay(S, 0.999)[:T]
    split = _run(q, k, v, m)
    f32 = _run(q, k, v, m, precise=True)
    qc, kc, vc, mc = (x.cuda().double() for x in (q, k, v, m))
    pm = (qc @ kc.T.contiguous()) * mc
    ref = pm @ vc
    bound = (pm.abs() @ vc.abs()) * 2.0 ** -20
    err_split = (split.cuda().double() - ref).abs()
    err_f32 = (f32.cuda().double() - ref).abs()
    assert bool((err_split <= bound + 1e-30).all()), float((err_split / bound).max())
    assert float(err_split.mean()) <= 1.25 * float(err_f32.mean())
    assert float(err_split.max()) <= 1e-5 * float(ref.abs().max())
    assert float(err_f32.max()) <= 1e-5 * float(ref.abs().max())


@pytest.mark.parametrize("split", [1, 2, 3, 7, 64])
def test_split_counts_and_determinism(split):
    g = torch.Generator().manual_seed(11)
    T, S, N, P = 300, 1000, 128, 128
    q = (torch.randn(T, N, generator=g) * N ** -0.5).half()
    k = (torch.randn(S, N, generator=g) * N ** -0.5).half()
    v = torch.randn(S, P, generator=g)
    m = _decay(S, 0.995)[:T]
    got = _run(q, k, v, m, split=split)
    check(got.numpy(), _want(q, k, v, m), False, 2e-3, f"split {split}")
    again = _run(q, k, v, m, split=split)
    assert torch.equal(got, again)


def test_zero_mask_and_strided_rows():
    g = torch.Generator().manual_seed(12)
    T, S, N, P = 128, 160, 64, 128
    qb = torch.randn(T, N + 8, generator=g).half()    # rows with a stride past N
    kb = torch.randn(S, N + 16, generator=g).half()
    q, k = qb[:, :N], kb[:, 4:4 + N]
    v = torch.randn(S, P, generator=g)
    m = torch.zeros(T, S)
    got = _run(q, k, v, m)
    assert torch.equal(got, torch.zeros(T, P))
    # Split partials of tiles that skipped every step are not stored and are
    # read back as +0: the sum stays +0 bit for bit (no -0).
    for split in (2, 5):
        got = _run(q, k, v, m, split=split)
        assert bool((got.view(torch.int32) == 0).all())
    m[5, 7] = 1.0   # one nonzero element: only row 5 is nonzero
    got = _run(q, k, v, m)
    check(got.numpy(), _want(q, k, v, m), False, 2e-3, "single nonzero")


def test_config5_full_size():
    """benchmark config 5's chain at full size (t = s = 4096, n = p = 128,
    gamma = 0.995): every element against a float64 GPU evaluation of the
    same chain, sampled rows against the oracle."""
    g = torch.Generator().manual_seed(6)
    s = 128 ** -0.5
    q = (torch.randn(4096, 128, generator=g) * s).half()
    k = (torch.randn(4096, 128, generator=g) * s).half()
    v = torch.randn(4096, 128, generator=g).half()
    m = _decay(4096, 0.995)
    got = _run(q, k, v, m)
    assert bool(torch.isfinite(got).all())
    qc, kc, vc, mc = (x.cuda().double() for x in (q, k, v, m))
    ref = ((qc @ kc.T.contiguous()) * mc) @ vc
    err = float((got.cuda().double() - ref).abs().max())
    assert err <= 2e-3 * float(ref.abs().max())
    rows = np.random.default_rng(0).integers(0, 4096, 24)
    want = oracle.linear_attention(q[rows].float().numpy(), k.float().numpy(), v.float().numpy(),
                                   m[rows].numpy())
    check(got[rows].numpy(), want, False, 2e-3, "config 5 rows")


def test_empty_s_gives_zeros():
    q = torch.randn(40, 16).half()
    got = _run(q, torch.zeros(0, 16).half(), torch.zeros(0, 24), torch.zeros(40, 0))
    assert torch.equal(got, torch.zeros(40, 24))


def test_rejects_bad_operands():
    from pto_einsum import linear_attention

    q = torch.zeros(4, 8, device="cuda", dtype=torch.float16)
    with pytest.raises(TypeError):
        linear_attention(q, q.float(), torch.zeros(4, 2, device="cuda"), torch.zeros(4, 4, device="cuda"))
    with pytest.raises(ValueError):
        linear_attention(q, q, torch.zeros(5, 2, device="cuda"), torch.zeros(4, 4, device="cuda"))
    with pytest.raises(RuntimeError):
        linear_attention(torch.zeros(4, 300, device="cuda", dtype=torch.float16),
                         torch.zeros(4, 300, device="cuda", dtype=torch.float16),
                         torch.zeros(4, 2, device="cuda"), torch.zeros(4, 4, device="cuda"))


def test_c_abi_misaligned_operands_use_the_workspace():
    """Through the C ABI: a q whose base is not 16-byte aligned is staged into
    the workspace; the size query (which assumes aligned bases) is then too
    small and the call fails cleanly, and succeeds with room for the copy."""
    import ctypes

    from pto_einsum import abi, runtime

    g = torch.Generator().manual_seed(13)
    T, S, N, P = 100, 96, 64, 128
    qb = (torch.randn(T * N + 8, generator=g) * 0.1).half().cuda()
    q = qb[2:2 + T * N].view(T, N)                     # base 4 bytes past a 16-byte boundary
    k = (torch.randn(S, N, generator=g) * 0.1).half().cuda()
    v = torch.randn(S, P, generator=g).cuda()
    m = _decay(max(T, S), 0.99)[:T, :S].contiguous().cuda()
    d = abi.LinAttnDesc()
    d.qk_dtype, d.v_dtype, d.m_dtype, d.split = 1, 0, 0, 1
    d.T, d.S, d.N, d.P = T, S, N, P
    d.q_ts, d.k_ss, d.v_ss, d.m_ts = N, N, P, S
    d.q_numel, d.k_numel, d.v_numel, d.m_numel = T * N, S * N, S * P, T * S
    lib = abi.bind()
    small = lib.pe_linear_attention_workspace_bytes(ctypes.byref(d))
    out = torch.empty(T, P, device="cuda")
    ws = torch.empty(small + (1 << 20), dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [ctypes.c_void_p(x.data_ptr()) for x in (q, k, v, m, out, ws)]
    rc = lib.pe_linear_attention(ctypes.byref(d), *args[:5], args[5], small, st)
    assert rc == -4 and "workspace" in runtime.last_error()
    rc = lib.pe_linear_attention(ctypes.byref(d), *args[:5], args[5], small + (1 << 20), st)
    assert rc == 0, runtime.last_error()
    check(out.cpu().numpy(), _want(q.cpu(), k.cpu(), v.cpu(), m.cpu()), False, 2e-3, "misaligned q")


@pytest.mark.parametrize("where", ["k", "v", "q"])
@pytest.mark.parametrize("precise", [False, True], ids=["split_pv", "f32_pv"])
def test_non_finite_operands_reach_masked_blocks(where, precise):
    """The chain of einsums turns an inf or NaN under a zero mask value into
    NaN (inf * 0); blocks whose mask is zero are skipped only when their
    q, k and v are finite, so the same outputs come out non-finite."""
    g = torch.Generator().manual_seed(13)
    T, S, N, P = 160, 160, 64, 96
    q = (torch.randn(T, N, generator=g) * N ** -0.5).half()
    k = (torch.randn(S, N, generator=g) * N ** -0.5).half()
    v = torch.randn(S, P, generator=g).half()
    m = _decay(S, 0.97)[:T]           # causal: m[t, s] = 0 for s > t
    if where == "k":
        k[150, 3] = float("inf")      # row s = 150 lies under a zero mask for t < 150
    elif where == "v":
        v[140, 7] = float("inf")
    else:
        q[10, 0] = float("nan")
    got = _run(q, k, v, m, precise=precise).numpy()
    want = _want(q, k, v, m)
    assert np.array_equal(np.isfinite(got), np.isfinite(want))
    assert not np.isfinite(want).all()
    fin = np.isfinite(want)
    if fin.any():
        err = float(np.abs(got[fin] - want[fin]).max())
        assert err <= 2e-3 * max(1.0, float(np.abs(want[fin]).max()))
