"""GPU parity of the decode-layer ops either side of the attention step against
the oracle: add_rms_norm_decode_raw_f16 (src/kernels.rs:3076-3216), the
GemvInPlace projections of the decode graph (src/cublas.rs:572-607) and the
two-stage greedy argmax (src/kernels.rs:345-505).

Contract:
* residual_out bit-exact (one f32 add of two f16 values, rounded once);
* the normalised output within 1 f16 ulp of the oracle (the sum of squares is
  reduced in a different order);
* GEMV within 1 f16 ulp plus twice the f32 accumulation bound
  k * 2^-24 * sum|w x| of the oracle's float64-checked result, and exact on
  row-selection matrices;
* argmax token bit-exact, including ties (lowest index), NaN (never chosen)
  and ragged lengths.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import f16_ulp_diff, normal_f16, rng

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _f16_ulp(v):
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.parametrize("n,eps,seed", [
    (5120, 1e-6, 1),     # Qwen3-32B hidden
    (2560, 1e-6, 2),     # Qwen3-4B hidden
    (1024, 1e-6, 3),     # Qwen3-0.6B hidden
    (8, 1e-6, 4),        # one 16-byte chunk
    (1000, 0.25, 5),     # ragged: the last wavefronts hold part of a chunk row
    (32768, 1e-6, 6),    # the one-workgroup maximum
])
def test_add_rms_norm_matches_oracle(gpu, n, eps, seed):
    import torch
    import grout_amd

    g = rng(1000 + seed)
    r, x = normal_f16(g, n, 2.0), normal_f16(g, n, 0.5)
    w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float16)
    dr, dx, dw = _dev(torch, r), _dev(torch, x), _dev(torch, w)
    out = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    res = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    grout_amd.add_rms_norm_decode(dr, dx, dw, out, res, eps)
    torch.cuda.synchronize()
    eo, er = oracle.add_rms_norm(r, x, w, eps)
    assert np.array_equal(res.cpu().numpy().view(np.uint16), er.view(np.uint16))
    d = f16_ulp_diff(out.cpu().numpy(), eo)
    assert d.max() <= 1, f"norm output {d.max()} ulp from the oracle"


def test_add_rms_norm_in_place_residual(gpu):
    """The decode graph writes residual_out over the residual input."""
    import torch
    import grout_amd

    g = rng(1010)
    n = 5120
    r, x = normal_f16(g, n), normal_f16(g, n)
    w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float16)
    dr, dx, dw = _dev(torch, r), _dev(torch, x), _dev(torch, w)
    out = torch.empty_like(dr)
    grout_amd.add_rms_norm_decode(dr, dx, dw, out, dr, 1e-6)
    torch.cuda.synchronize()
    eo, er = oracle.add_rms_norm(r, x, w, 1e-6)
    assert np.array_equal(dr.cpu().numpy().view(np.uint16), er.view(np.uint16))
    assert f16_ulp_diff(out.cpu().numpy(), eo).max() <= 1


def _gemv_check(got, w, x, ref):
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    bound = _f16_ulp(ref) + 2 * w.shape[1] * 2.0 ** -24 * (np.abs(w64) @ np.abs(x64))
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= bound), f"gemv: max err {err.max():.3e}"
    return float(err.max())


@pytest.mark.parametrize("m,k,seed", [
    (10240, 5120, 1),    # Qwen3-32B merged qkv_proj (64 + 2*8 heads of 128)
    (5120, 8192, 2),     # Qwen3-32B o_proj
    (6144, 2560, 3),     # Qwen3-4B merged qkv_proj
    (17, 8, 4),          # ragged rows, k = one chunk
    (100, 24, 5),        # k below one wavefront's chunk row
    (33, 1032, 6),       # k not a multiple of the unrolled chunk row
    (3, 32768, 7),       # the LDS maximum of x
])
def test_gemv_matches_oracle(gpu, m, k, seed):
    import torch
    import grout_amd

    g = rng(1100 + seed)
    w = normal_f16(g, (m, k), 1.0 / math.sqrt(k))
    x = normal_f16(g, k)
    out = torch.full((m,), float("nan"), dtype=torch.float16, device="cuda")
    grout_amd.gemv_f16(_dev(torch, w), _dev(torch, x), out)
    torch.cuda.synchronize()
    _gemv_check(out.cpu().numpy(), w, x, oracle.gemv_f16(w, x))


def test_gemv_row_selection_exact(gpu):
    import torch
    import grout_amd

    g = rng(1120)
    m, k = 1000, 520
    perm = g.integers(0, k, m)
    w = np.zeros((m, k), np.float16)
    w[np.arange(m), perm] = 1.0
    x = normal_f16(g, k)
    out = torch.empty((m,), dtype=torch.float16, device="cuda")
    grout_amd.gemv_f16(_dev(torch, w), _dev(torch, x), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), x[perm])


def _argmax_gpu(torch, lg):
    import grout_amd

    d = _dev(torch, lg)
    bm, bi = grout_amd.argmax_scratch(lg.shape[0])
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    grout_amd.argmax_f16(d, bm, bi, tok)
    torch.cuda.synchronize()
    return int(tok.cpu().numpy().view(np.uint32)[0])


@pytest.mark.parametrize("n", [1, 7, 2048, 2049, 100003, 151936])
def test_argmax_matches_oracle(gpu, n):
    import torch

    g = rng(1200 + n % 97)
    lg = normal_f16(g, n, 4.0)
    assert _argmax_gpu(torch, lg) == oracle.argmax_f16(lg) == int(np.argmax(lg))


def test_argmax_ties_nan_inf(gpu):
    import torch

    g = rng(1230)
    n = 151936
    lg = normal_f16(g, n)
    lg[[150000, 90000, 5000]] = np.float16(30.0)   # ties in three blocks
    assert _argmax_gpu(torch, lg) == oracle.argmax_f16(lg) == 5000
    lg[[5001, 5002]] = np.float16(30.0)            # ties inside one block
    lg[4096] = np.float16(np.nan)
    lg[0] = np.float16(-np.inf)
    assert _argmax_gpu(torch, lg) == oracle.argmax_f16(lg) == 5000
    lg[7] = np.float16(np.inf)
    assert _argmax_gpu(torch, lg) == oracle.argmax_f16(lg) == 7
    for fill in (-np.inf, np.nan, 0.0):
        z = np.full(5000, fill, np.float16)
        assert _argmax_gpu(torch, z) == oracle.argmax_f16(z) == 0
