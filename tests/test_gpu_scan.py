"""Parity of the linear-recurrence scan kernels (ppo_linear_scan_fwd/bwd,
boonta_amd/kernels/scan.py) against the float64 oracle (oracle/scan.py),
following the reference's tests/test_networks.py:141-209.

Tolerances (written here): float32 storage — forward atol 1e-5 (rtol 1e-5),
gradients atol 1e-4 (the reference's own bounds); bf16 storage — forward
within 1e-2 of the exact float32 result of the bf16 inputs, and on the
64-step problem a relative error at most bf16's machine epsilon and below
that of a scan that accumulates in bf16; bf16 gradients 2e-2 relative.
The SSM block's reset (networks/blocks/ssm.py:40-55) folded into the same
launches: float32 1e-5 (gradients atol 1e-4), bf16 2e-2, against the oracle's
masking + scan; with no dones it is bit-identical to the plain scan."""
import numpy as np
import pytest
import torch

from boonta_amd import _lib
from boonta_amd.kernels import get_scan_implementation, hip, scan, ssm, ssm_scan
from oracle import scan as oscan

pytestmark = pytest.mark.gpu

BF16_EPS = 2.0 ** -7


def problem(seed, shape, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(shape, generator=g) * 0.9 + 0.05
    b = torch.rand(shape, generator=g)
    init = torch.randn((shape[0], shape[-1]), generator=g)
    return tuple(x.to(dtype).cuda() for x in (a, b, init))


def np64(x):
    return x.detach().float().cpu().numpy().astype(np.float64)


def test_the_scan_matches_the_reference_and_its_gradients():
    a, b, init = problem(3, (4, 16, 128))
    for x in (a, b, init):
        x.requires_grad_(True)
    out = scan(a, b, init)
    want = oscan.forward(np64(a), np64(b), np64(init))
    np.testing.assert_allclose(np64(out), want, rtol=1e-5, atol=1e-5)
    w = torch.randn(a.shape, generator=torch.Generator().manual_seed(4)).cuda()
    (out * w).sum().backward()
    da, db, dinit = oscan.vjp(np64(a), want, np64(init), np64(w))
    for got, exp in ((a.grad, da), (b.grad, db), (init.grad, dinit)):
        np.testing.assert_allclose(np64(got), exp, atol=1e-4)


@pytest.mark.parametrize("steps", [1, 7, 8, 9, 17, 63, 64, 200])
@pytest.mark.parametrize("features,batch", [(1, 3), (3, 2), (4, 1), (100, 2), (256, 8), (1024, 1)])
def test_ragged_shapes_and_time_chunks(steps, features, batch):
    a, b, init = problem(steps * 1000 + features, (batch, steps, features))
    out = torch.empty_like(a)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("ppo_linear_scan_fwd", st, 0, a.data_ptr(), b.data_ptr(), init.data_ptr(), out.data_ptr(), batch,
              steps, features)
    want = oscan.forward(np64(a), np64(b), np64(init))
    np.testing.assert_allclose(np64(out), want, rtol=1e-5, atol=1e-5)
    g = torch.randn(a.shape, generator=torch.Generator().manual_seed(steps)).cuda()
    da, db, dinit = torch.empty_like(a), torch.empty_like(a), torch.empty_like(init)
    _lib.call("ppo_linear_scan_bwd", st, 0, a.data_ptr(), out.data_ptr(), init.data_ptr(), g.data_ptr(),
              da.data_ptr(), db.data_ptr(), dinit.data_ptr(), batch, steps, features)
    eda, edb, edinit = oscan.vjp(np64(a), np64(out), np64(init), np64(g))
    np.testing.assert_allclose(np64(db), edb, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np64(da), eda, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np64(dinit), edinit, rtol=1e-5, atol=1e-5)


def test_widths_the_vector_loads_cannot_tile_still_scan_in_bf16():
    a, b, init = problem(6, (2, 8, 100), torch.bfloat16)
    out = get_scan_implementation("hip")(a, b, init)
    assert out.dtype == torch.bfloat16
    np.testing.assert_allclose(np64(out), oscan.forward(np64(a), np64(b), np64(init)), rtol=1e-2, atol=1e-2)


def test_bf16_storage_accumulates_in_single_precision():
    a, b, init = problem(5, (8, 64, 256), torch.bfloat16)
    out = np64(scan(a, b, init))
    exact = oscan.forward(np64(a), np64(b), np64(init))
    assert np.max(np.abs(out - exact) / np.abs(exact)) <= BF16_EPS
    # a scan that rounds its carry to bf16 every step drifts further
    h = np64(init)
    drifted = np.empty_like(exact)
    A, B = np64(a), np64(b)
    to_bf16 = lambda x: torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    for t in range(A.shape[1]):
        h = to_bf16(to_bf16(A[:, t] * h) + B[:, t])
        drifted[:, t] = h
    assert np.abs(out - exact).max() < np.abs(drifted - exact).max()


def test_bf16_gradients():
    a, b, init = problem(7, (4, 32, 128), torch.bfloat16)
    for x in (a, b, init):
        x.requires_grad_(True)
    out = scan(a, b, init)
    w = torch.randn(a.shape, generator=torch.Generator().manual_seed(8)).cuda().to(torch.bfloat16)
    (out.float() * w.float()).sum().backward()
    assert a.grad.dtype == torch.bfloat16 and init.grad.dtype == torch.bfloat16
    da, db, dinit = oscan.vjp(np64(a), np64(out), np64(init), np64(w))
    for got, exp in ((a.grad, da), (b.grad, db), (init.grad, dinit)):
        err = np.linalg.norm(np64(got) - exp) / np.linalg.norm(exp)
        assert err < 2e-2, err


def test_a_scan_that_stores_half_returns_half():
    half = torch.full((4, 16, 128), 0.5, dtype=torch.bfloat16, device="cuda")
    init = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")
    assert scan(half, half, init).dtype == torch.bfloat16


def test_extra_axes_fold_into_the_batch():
    a, b, _ = problem(9, (2, 12, 3, 16))
    init = torch.randn(2, 3, 16, generator=torch.Generator().manual_seed(1)).cuda()
    out = hip(a, b, init)
    assert out.shape == a.shape
    fa = np64(a).transpose(0, 2, 1, 3).reshape(6, 12, 16)
    fb = np64(b).transpose(0, 2, 1, 3).reshape(6, 12, 16)
    want = oscan.forward(fa, fb, np64(init).reshape(6, 16)).reshape(2, 3, 12, 16).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(np64(out), want, rtol=1e-5, atol=1e-5)


def test_large_scan_is_linear_and_matches_a_chunk_of_the_oracle():
    """Size-independent checks at a bandwidth-sized shape: linearity in (b,
    init), and the oracle on a slice of the batch."""
    a, b, init = problem(10, (512, 64, 512))
    _, b2, init2 = problem(11, (512, 64, 512))
    h1, h2 = scan(a, b, init), scan(a, b2, init2)
    h12 = scan(a, b + b2, init + init2)
    torch.testing.assert_close(h12, h1 + h2, rtol=1e-5, atol=1e-5)
    want = oscan.forward(np64(a[:8]), np64(b[:8]), np64(init[:8]))
    np.testing.assert_allclose(np64(h1[:8]), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("steps", [1, 9, 16, 64, 200])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_reset", [False, True])
def test_ssm_reset_matches_the_oracle(steps, dtype, with_reset):
    """networks/blocks/ssm.py:40-55: episode starts restart the recurrence
    from the cell's initial carry, folded into the scan launches."""
    batch, features = 6, 128
    a, b, carry = problem(steps + 17, (batch, steps, features), dtype)
    g = torch.Generator().manual_seed(steps)
    done = (torch.rand((batch, steps), generator=g) < 0.2)
    done[0, 0] = True
    done = done.cuda()
    reset = torch.randn((batch, features), generator=g).to(dtype).cuda() if with_reset else None
    for x in (a, b, carry):
        x.requires_grad_(True)
    final, carries = ssm(a, b, done, carry, reset)
    assert carries.dtype == dtype and final.shape == carry.shape
    dn = done.cpu().numpy()
    rn = None if reset is None else np64(reset)
    want = oscan.ssm_forward(np64(a), np64(b), dn, np64(carry), rn)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    np.testing.assert_allclose(np64(carries), want, rtol=tol, atol=tol)
    np.testing.assert_array_equal(np64(final), np64(carries)[:, -1])
    w = torch.randn(a.shape, generator=g).cuda().to(dtype)
    (carries.float() * w.float()).sum().backward()
    da, db, dc = oscan.ssm_vjp(np64(a), np64(carries), dn, np64(carry), np64(w), rn)
    for got, exp in ((a.grad, da), (b.grad, db), (carry.grad, dc)):
        if dtype == torch.float32:
            np.testing.assert_allclose(np64(got), exp, rtol=1e-5, atol=1e-4)
        else:
            err = np.linalg.norm(np64(got) - exp) / max(np.linalg.norm(exp), 1e-12)
            assert err < 2e-2, err


def test_ssm_without_dones_is_the_plain_scan():
    a, b, carry = problem(21, (4, 64, 256))
    done = torch.zeros((4, 64), dtype=torch.bool, device="cuda")
    torch.testing.assert_close(ssm_scan(a, b, done, carry), scan(a, b, carry), rtol=0, atol=0)
