"""HIP kernels of the layer pipeline (include/exl3_layer.h) against float64
numpy: the blockwise Hadamard transform (hadamard.py:73-126) against the
Sylvester matrix product, block_rms (regularize.py:41-56) against a float64
sum of squares, and the blocked Cholesky (cholesky_ex, the factorisation of
block_ldl, ldlq.py:76-142) against numpy.linalg.cholesky, including the
failure index of matrices that are not positive definite."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import ldlq_ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _sylvester64(n=128):
    i = np.arange(n)
    pop = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pop % 2 == 0, 1.0, -1.0) / np.sqrt(n)


def _blockwise_left(x, h):
    k, n = x.shape
    return np.einsum("ij,bjn->bin", h, x.reshape(k // 128, 128, n)).reshape(k, n)


@pytest.mark.parametrize("shape", [(128, 128), (256, 384), (384, 1000), (1024, 128)])
def test_hadamard128_matches_sylvester_product(torch_mod, shape):
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd import hadamard
    rng = np.random.default_rng(sum(shape))
    k, n = shape
    x = rng.standard_normal((k, n)).astype(np.float32)
    h = _sylvester64()
    np.testing.assert_allclose(h, ldlq_ref.hadamard(), rtol=0, atol=1e-7)
    xt = torch.from_numpy(x).cuda()
    want_l = _blockwise_left(x.astype(np.float64), h)
    got_l = hadamard.preapply_had_l(xt).cpu().numpy()
    np.testing.assert_allclose(got_l, want_l, rtol=0, atol=2e-6 * np.abs(want_l).max())
    if n % 128 == 0:
        want_r = _blockwise_left(x.astype(np.float64).T, h).T
        got_r = hadamard.preapply_had_r(xt).cpu().numpy()
        np.testing.assert_allclose(got_r, want_r, rtol=0, atol=2e-6 * np.abs(want_r).max())
        # In place, and the transform is its own inverse.
        y = xt.clone()
        hadamard.blockwise_preapply_had_r_(y)
        assert np.array_equal(y.cpu().numpy(), got_r)
        hadamard.blockwise_preapply_had_r_(y)
        np.testing.assert_allclose(y.cpu().numpy(), x, rtol=0, atol=1e-5)
    else:
        with pytest.raises(ValueError, match="divisible"):
            hadamard.preapply_had_r(xt)
    y = xt.clone()
    hadamard.blockwise_preapply_had_l_(y)
    assert np.array_equal(y.cpu().numpy(), got_l)
    # A unit vector maps to a signed column of the matrix.
    e = torch.zeros((128, n), device="cuda")
    e[5, 3] = 1.0
    col = hadamard.preapply_had_l(e).cpu().numpy()[:, 3]
    np.testing.assert_allclose(col, h[:, 5], rtol=0, atol=1e-7)


def test_hadamard128_rejects_bad_shapes(torch_mod):
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd import _native
    x = torch.zeros((100, 128), device="cuda")
    with pytest.raises(RuntimeError, match="divisible by 128"):
        _native.hadamard128(x, x, 0)
    with pytest.raises(RuntimeError, match="side"):
        _native.hadamard128(x, x, 2)
    with pytest.raises(RuntimeError, match="shape"):
        _native.hadamard128(x, torch.zeros((100, 64), device="cuda"), 1)


@pytest.mark.parametrize("shape,blocksize", [((256, 384), 32), ((100, 70), 32), ((33, 1000), 7)])
def test_block_rms_matches_float64(torch_mod, shape, blocksize):
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.regularize import block_rms
    rng = np.random.default_rng(shape[0])
    x = (rng.standard_normal(shape) * rng.uniform(0.1, 10, size=shape[1])).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    for dim in (0, 1):
        want = np.sqrt((x.astype(np.float64) ** 2).mean(axis=dim))
        got = block_rms(xt, dim=dim, keepdim=True, blocksize=blocksize)
        assert tuple(got.shape) == ((1, shape[1]) if dim == 0 else (shape[0], 1))
        np.testing.assert_allclose(got.cpu().numpy().ravel(), want, rtol=2e-6)
    # Slice order: a single 32-slice equals the plain sequential sum.
    z = torch.zeros((32, 3), device="cuda")
    z[:, 1] = 2.0
    np.testing.assert_array_equal(block_rms(z, dim=0).cpu().numpy(), [0.0, 2.0, 0.0])


def _spd(n, seed, cond_shift=0.05):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n + 8, n))
    X[:, rng.random(n) < 0.05] *= 10.0
    return ((X.T @ X) / (n + 8) + cond_shift * np.eye(n)).astype(np.float32)


@pytest.mark.parametrize("n", [1, 5, 128, 129, 300, 512])
def test_cholesky_matches_numpy(torch_mod, n):
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.ldlq import cholesky_ex
    A = _spd(n, n)
    # Upper-triangle garbage must not be read.
    A_in = A.copy()
    A_in[np.triu_indices(n, 1)] = 7.0
    L, info = cholesky_ex(torch.from_numpy(A_in).cuda())
    assert int(info.item()) == 0
    Lh = L.cpu().numpy()
    assert not np.any(np.triu(Lh, 1)), "non-zero above the diagonal"
    want = np.linalg.cholesky(A.astype(np.float64))
    np.testing.assert_allclose(Lh, want, rtol=0, atol=5e-5 * np.abs(want).max())
    resid = np.linalg.norm(A - Lh.astype(np.float64) @ Lh.T.astype(np.float64)) / np.linalg.norm(A)
    assert resid < 2e-6, resid


@pytest.mark.parametrize("n,bad", [(64, 0), (300, 2), (300, 200), (512, 511)])
def test_cholesky_failure_index(torch_mod, n, bad):
    """info = 1-based order of the first leading minor that is not positive
    definite, as torch.linalg.cholesky_ex reports it."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.ldlq import cholesky_ex
    A = np.eye(n, dtype=np.float32)
    A[bad, bad] = -1.0
    _, info = cholesky_ex(torch.from_numpy(A).cuda())
    assert int(info.item()) == bad + 1
    _, info_t = torch.linalg.cholesky_ex(torch.from_numpy(A).double())
    assert int(info_t) == bad + 1
    A = _spd(n, 3)
    A[bad, bad] = float("nan")
    _, info = cholesky_ex(torch.from_numpy(A).cuda())
    assert int(info.item()) == bad + 1


def test_block_ldl_damping_retries_on_gpu(torch_mod):
    """A matrix just below positive definite fails once, is damped by
    2 sigma mean(diag) (ldlq.py:96-104) and factors; the folded factor has
    identity diagonal blocks and matches the numpy oracle."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.ldlq import block_ldl
    A = _spd(256, 9).astype(np.float64)
    w_min = np.linalg.eigvalsh(A)[0]
    A = (A - (w_min + 1e-3) * np.eye(256)).astype(np.float32)
    res = block_ldl(torch.from_numpy(A).cuda())
    assert res.retries >= 1 and res.damping_applied
    ref_T, _, ref_retries = ldlq_ref.block_ldl(A)
    assert res.retries == ref_retries
    T = res.transformed.cpu().numpy()
    for b in range(16):
        np.testing.assert_array_equal(T[16 * b:16 * b + 16, 16 * b:16 * b + 16], np.eye(16))
    np.testing.assert_allclose(T, ref_T, rtol=0, atol=5e-4 * np.abs(ref_T).max())


@pytest.mark.parametrize("shapes", [[(256, 128)], [(256, 128), (128, 256), (384, 384)]])
def test_fused_ldlq_steps_match_host_traversal(torch_mod, shapes):
    """exl3_ldlq_gather / exl3_ldlq_scatter (the GPU traversal) against the
    torch traversal on the CPU, one problem and three in lockstep
    (ldlq.py:163-309). The stand-in encoder halves its tiles (a continuous
    map, so GEMM rounding differences stay at fp32 level) and returns states
    that encode each element's batch position and call number, so every
    state must land in the same place exactly."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.ldlq import ldlq_lockstep
    probs = []
    for s, (k, n) in enumerate(shapes):
        rng = np.random.default_rng(100 + s)
        W = rng.standard_normal((k, n)).astype(np.float32)
        X = rng.standard_normal((4 * k, k)).astype(np.float32)
        H = (X.T @ X) / np.float32(X.shape[0]) + np.float32(0.05) * np.eye(k, dtype=np.float32)
        L, _, _ = ldlq_ref.block_ldl(H)
        probs.append((W, L))
    seen = {"cpu": [], "gpu": []}

    def recorder(key):
        def enc(tiles):
            call = len(seen[key])
            seen[key].append(tiles.cpu().clone())
            pos = torch.arange(tiles.numel(), device=tiles.device).view(tiles.shape)
            return tiles * 0.5, ((pos * 7 + call) & 0x7FFF).to(torch.int16)
        return enc

    cpu = ldlq_lockstep([(torch.from_numpy(W), torch.from_numpy(L)) for W, L in probs],
                        recorder("cpu"), buf_size_k=64)
    gpu = ldlq_lockstep([(torch.from_numpy(W).cuda(), torch.from_numpy(L).cuda())
                         for W, L in probs], recorder("gpu"), buf_size_k=64)
    assert len(seen["cpu"]) == len(seen["gpu"]) == max(k for k, _ in shapes) // 16
    for a, b in zip(seen["cpu"], seen["gpu"]):
        np.testing.assert_allclose(b.numpy(), a.numpy(), rtol=0, atol=1e-4)
    for c, g in zip(cpu, gpu):
        np.testing.assert_allclose(g.weight_q.cpu().numpy(), c.weight_q.numpy(), rtol=0,
                                   atol=1e-4)
        assert torch.equal(g.encoded.cpu(), c.encoded)
        assert g.encoder_calls == c.encoder_calls


def _ldlq_call(torch, widths, seed):
    """Device matrices of one LDLQ encoder call over blocks of the given
    widths (16 rows each) and its exl3_ldlq_block table."""
    from exl3_intel_arc_quantizer_amd import _native
    rng = np.random.default_rng(seed)
    blocks, rows, tile0 = [], [], 0
    for n in widths:
        W = torch.from_numpy(rng.standard_normal((16, n)).astype(np.float32) * 3).cuda()
        C = torch.from_numpy(rng.standard_normal((16, n)).astype(np.float32)).cuda()
        Wq = torch.full((16, n), 7.0, device="cuda")
        E = torch.full((16, n), 7.0, device="cuda")
        S = torch.zeros((n // 16, 256), dtype=torch.int16, device="cuda")
        blocks.append((W, C, Wq, E, S))
        rows.append([W.data_ptr(), C.data_ptr(), Wq.data_ptr(), E.data_ptr(), S.data_ptr(), n,
                     tile0, 0])
        tile0 += n // 16
    _native.check_ldlq_rows(rows, tile0)
    table = torch.tensor(rows, dtype=torch.int64, device="cuda")
    return blocks, table, tile0


def _tiles_of(torch, m, perm):
    """(n / 16, 256) tiles of a 16 x n matrix in tensor-core order: element p
    of tile t is m[perm[p] // 16][16 t + perm[p] % 16]."""
    n = m.shape[1]
    t = m.reshape(16, n // 16, 16).permute(1, 0, 2).reshape(n // 16, 256)
    return t[:, torch.from_numpy(perm).to(m.device)]


@pytest.mark.parametrize("widths", [[16 * 5], [16 * 3, 16 * 21, 16 * 9], [16 * 8, 16 * 16]])
def test_ldlq_gather_and_scatter_kernels(torch_mod, widths):
    """exl3_ldlq_gather against the tensor-core tiles of W + compensation
    (NaN and inf - inf sums included), and exl3_ldlq_scatter's Wq, E and
    states at the same places, for calls of one block and of several blocks
    of different widths."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd import _native
    from oracle import trellis_format_ref
    perm = trellis_format_ref.tensor_core_perm()
    blocks, table, tiles = _ldlq_call(torch, widths, sum(widths))
    W0, C0 = blocks[0][0], blocks[0][1]
    W0[3, 5] = float("nan")
    W0[15, widths[0] - 1] = float("inf")
    C0[15, widths[0] - 1] = float("-inf")
    want = torch.cat([_tiles_of(torch, W + C, perm) for W, C, *_ in blocks])
    x = torch.full((tiles, 256), -5.0, device="cuda")
    _native.ldlq_gather(table, x)
    assert torch.equal(x.isnan(), want.isnan()) and int(x.isnan().sum()) == 2
    assert torch.equal(torch.nan_to_num(x), torch.nan_to_num(want))

    gen = torch.Generator(device="cpu").manual_seed(7)
    recon = torch.randn((tiles, 256), generator=gen).half().float().cuda()
    idx = torch.randint(-32768, 32767, (tiles, 256), generator=gen, dtype=torch.int16).cuda()
    _native.ldlq_scatter(table, recon, idx)
    t0 = 0
    for W, C, Wq, E, S in blocks:
        nt = W.shape[1] // 16
        assert torch.equal(_tiles_of(torch, Wq, perm), recon[t0:t0 + nt])
        diff = _tiles_of(torch, W, perm) - recon[t0:t0 + nt]
        got = _tiles_of(torch, E, perm)
        assert torch.equal(got.isnan(), diff.isnan())
        assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(diff))
        assert torch.equal(S, idx[t0:t0 + nt])
        t0 += nt


def test_hessian_from_half_activations_matches_float32(torch_mod):
    """calibration.py:337-385 on bf16 / fp16 activations: the half-precision
    GEMM with float32 output equals the float32 GEMM of the converted
    values up to summation order (float64 reference), damping included."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.layer_quant import hessian_from_activations
    rng = np.random.default_rng(5)
    X = rng.standard_normal((3000, 384)).astype(np.float32)
    X[:, rng.random(384) < 0.05] *= 10.0
    for dt in (torch.bfloat16, torch.float16):
        xh = torch.from_numpy(X).to(dt)
        x64 = xh.double().numpy()
        want = x64.T @ x64 / x64.shape[0]
        H, damp = hessian_from_activations(xh.cuda(), chunk_tokens=1024)
        H32, damp32 = hessian_from_activations(xh.float().cuda(), chunk_tokens=1024)
        want_damp = 0.01 * np.diag(want).mean()
        # Both paths against float64 (the float32 GEMM of the converted
        # values measured ~2e-6 relative error here, the half-precision one
        # ~1e-7).
        assert damp == pytest.approx(want_damp, rel=1e-5)
        assert damp32 == pytest.approx(want_damp, rel=1e-5)
        want[np.diag_indices(384)] += want_damp
        scale = np.abs(want).max()
        np.testing.assert_allclose(H.cpu().numpy(), want, rtol=0, atol=1e-5 * scale)
        np.testing.assert_allclose(H32.cpu().numpy(), want, rtol=0, atol=1e-5 * scale)


@pytest.mark.parametrize("shape", [(128, 128), (256, 384), (384, 1024)])
def test_hadamard128_scaled_equals_divide_then_transform(torch_mod, shape):
    """exl3_hadamard128_scaled (the fused folds of regularize.py:159-173):
    bit for bit the torch division followed by exl3_hadamard128, on both
    sides and in place; the row slice sums of squares equal float64 sums
    of the transformed rows' 32-element slices."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd import _native, hadamard
    k, n = shape
    rng = np.random.default_rng(k + n)
    x = torch.from_numpy(rng.standard_normal((k, n)).astype(np.float32)).cuda()
    dcol = torch.from_numpy((rng.random(n) * 3 + 0.1).astype(np.float32)).cuda()
    drow = torch.from_numpy((rng.random(k) * 3 - 1.6).astype(np.float32)).cuda()
    out = torch.empty_like(x)
    sq = torch.empty((k, n // 32), dtype=torch.float32, device="cuda")
    _native.hadamard128_scaled(x, out, 1, divisor=dcol, slice_sumsq=sq)
    want = hadamard.preapply_had_r(x / dcol.reshape(1, n))
    assert torch.equal(out, want)
    o64 = want.cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(sq.cpu().numpy(), (o64 ** 2).reshape(k, n // 32, 32).sum(-1),
                               rtol=2e-6)
    _native.hadamard128_scaled(x, out, 0, divisor=drow)
    assert torch.equal(out, hadamard.preapply_had_l(x / drow.reshape(k, 1)))
    y = x.clone()
    _native.hadamard128_scaled(y, y, 0, divisor=drow)
    assert torch.equal(y, out)
    _native.hadamard128_scaled(x, out, 1)
    assert torch.equal(out, hadamard.preapply_had_r(x))
    rms = torch.empty(k, dtype=torch.float32, device="cuda")
    _native.block_rms_from_slices(sq, rms, n)
    np.testing.assert_allclose(rms.cpu().numpy(), np.sqrt((o64 ** 2).mean(axis=1)), rtol=2e-6)
    with pytest.raises(RuntimeError):                           # wrong length for side 0
        _native.hadamard128_scaled(x, out, 0, divisor=torch.ones(k + 1, device="cuda"))
    with pytest.raises(RuntimeError):
        _native.hadamard128_scaled(x, out, 0, slice_sumsq=sq)    # sums only with side 1


@pytest.mark.parametrize("name", ["columns", "tiny", "dead", "skew_below", "skew_above"])
def test_regularize_closed_forms_gpu(torch_mod, name):
    """The product's regularize (three passes over the fused kernels) gives
    the scale values the definition fixes (tests/regularize_cases.py), the
    flag and skew, and decodes back to W."""
    torch = torch_mod
    from exl3_intel_arc_quantizer_amd.hadamard import weight_from_quantized
    from exl3_intel_arc_quantizer_amd.regularize import regularize

    from .regularize_cases import K, N, cases, check
    case = cases()[name]
    W = torch.from_numpy(case["W"]).cuda()
    args = {}
    res = regularize(W, torch.ones((K, 1), device="cuda"), torch.ones((1, N), device="cuda"),
                     quant_args=args, H_diag=torch.from_numpy(case["H_diag"]).cuda())
    assert torch.equal(W, torch.from_numpy(case["W"]).cuda())          # input untouched
    assert args["zeros"] is False and res.zeros is False
    if "skew" in case["expected"]:
        assert res.skew_factor == pytest.approx(case["expected"]["skew"], rel=1e-5)
    back = weight_from_quantized(res.weight, res.su, res.sv)
    check(name, case, res.weight.cpu().numpy(), res.su.cpu().numpy(), res.sv.cpu().numpy(),
          res.apply_out_scales, back.cpu().numpy())
    if name == "dead":
        assert res.out_channel_scales[0, 5].item() == pytest.approx(0.1)
    # Forced flags and the all-zero weight (quant_args["zeros"]).
    z = regularize(torch.zeros((K, N), device="cuda"), torch.ones((K, 1), device="cuda"),
                   torch.ones((1, N), device="cuda"), quant_args={"apply_out_scales": False})
    assert z.zeros and z.apply_out_scales and torch.count_nonzero(z.weight) == 0
    assert torch.count_nonzero(z.sv) == 0
    off = regularize(W, torch.ones((K, 1), device="cuda"), torch.ones((1, N), device="cuda"),
                     quant_args={"apply_out_scales": False},
                     H_diag=torch.from_numpy(case["H_diag"]).cuda())
    assert not off.apply_out_scales
