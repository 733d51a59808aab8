"""Cross entropy (fused log-softmax + NLL) against the oracle's restatement of
Spar's CPU path (loss/cross_entropy.cpp), and the reference-compatible NLL
entry points against exact gathers and scatters.

Tolerances: each loss is -lp at the target, so it carries log-softmax's
bound, |d lp| <= 1e-6 sqrt(C) + 4 eps (|lp| + log C + 1); a mean or sum of N
losses adds red(N).  The logits gradient g - exp(lp) g_t moves by
|g_t| exp(lp) (|d lp| + 4 eps) plus its own rounding.
"""
import numpy as np
import pytest

import oracle.reference as R
from tests.helpers import assert_bitexact, assert_ulp

pytestmark = pytest.mark.gpu

F32, F64 = np.float32, np.float64


@pytest.fixture(scope="module")
def sp():
    from spar_amd import spar

    if spar.hip_device_count() < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return spar


def reduction_of(sp, name):
    return {"none": sp.loss.Reduction.None_, "sum": sp.loss.Reduction.Sum,
            "mean": sp.loss.Reduction.Mean}[name]


def lp_bound(lp, classes, dtype):
    eps = np.finfo(dtype).eps
    return 1e-6 * np.sqrt(classes) + 4 * eps * (np.abs(lp) + np.log(classes) + 1)


def closed_lp(x):
    x = x.astype(np.float64)
    z = x - x.max(axis=-1, keepdims=True)
    return z - np.log(np.exp(z).sum(axis=-1, keepdims=True))


def run_both(sp, x, t, reduction, language_model=False):
    device, cpu = sp.Device.hip(0), sp.Device.cpu()
    logits = sp.Tensor.from_numpy(x).to(device)
    logits.set_requires_grad(True)
    targets = sp.Tensor.from_numpy(t).to(device)
    fn = sp.loss.language_model_cross_entropy if language_model else sp.loss.cross_entropy
    loss = fn(logits, targets, reduction_of(sp, reduction))
    (sp.sum(loss) if reduction == "none" else loss).backward()
    ref_logits = R.RTensor.of(x, requires_grad=True)
    ref_fn = R.language_model_cross_entropy if language_model else R.cross_entropy
    ref_loss = ref_fn(ref_logits, t, reduction)
    (R.sum(ref_loss) if reduction == "none" else ref_loss).backward()
    return (loss.to(cpu).numpy(), ref_loss.numpy(), logits.grad().to(cpu).numpy(),
            ref_logits.grad().numpy())


def check(got_loss, want_loss, got_dx, want_dx, x, per_row_targets, reduction, dtype, what):
    classes = x.shape[-1]
    lp = closed_lp(x)
    picked = -np.take_along_axis(lp, per_row_targets[..., None], -1)[..., 0]
    tol = lp_bound(picked, classes, dtype)
    count = picked.size
    if reduction == "none":
        err = np.abs(got_loss.astype(np.float64) - want_loss)
        assert np.all(err <= tol), f"{what} losses: worst excess {np.max(err - tol)}"
        upstream = 1.0
    else:
        total_tol = np.sum(tol) + 1e-6 * np.sqrt(count) * max(abs(float(want_loss.sum())),
                                                               float(np.sqrt(np.sum(picked ** 2))))
        if reduction == "mean":
            total_tol /= count
        assert abs(float(got_loss) - float(want_loss)) <= total_tol, f"{what} reduced loss"
        upstream = 1.0 / count if reduction == "mean" else 1.0
    eps = np.finfo(dtype).eps
    bound = (upstream * np.exp(lp) * (lp_bound(lp, classes, dtype) + 4 * eps)
             + 4 * eps * np.abs(want_dx) + np.finfo(dtype).tiny)
    err = np.abs(got_dx.astype(np.float64) - want_dx)
    assert np.all(err <= bound), f"{what} dlogits: worst excess {np.max(err - bound)}"


@pytest.mark.parametrize("dtype", [F32, F64])
@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_cross_entropy_matches_oracle(sp, dtype, reduction):
    """Class counts cover the fused forward's batch paths (float32 batches of
    8192 classes per workgroup): none whole (1000, 4096), one whole batch
    alone (8192) or with a partial tail (8292), two (16384), three with a
    tail (32000), and odd counts that take scalar loads (5, 50257)."""
    rng = np.random.default_rng(80)
    for rows, classes in [(1, 1), (3, 5), (64, 1000), (8, 4096), (3, 8192), (2, 8292),
                          (2, 16384), (4, 32000), (3, 50257)]:
        x = (rng.standard_normal((rows, classes)) * 2).astype(dtype)
        t = rng.integers(0, classes, rows).astype(np.int64 if rows % 2 else np.int32)
        got, want, gdx, wdx = run_both(sp, x, t, reduction)
        check(got, want, gdx, wdx, x, t.astype(np.int64), reduction, dtype,
              f"{rows}x{classes} {np.dtype(dtype).name} {reduction}")


def test_cross_entropy_batched_targets(sp):
    rng = np.random.default_rng(81)
    x = rng.standard_normal((4, 6, 37)).astype(F32)
    t = rng.integers(0, 37, (4, 6)).astype(np.int64)
    got, want, gdx, wdx = run_both(sp, x, t, "none")
    check(got, want, gdx, wdx, x, t, "none", F32, "[4,6,37]")


@pytest.mark.parametrize("reduction", ["none", "mean"])
def test_language_model_cross_entropy(sp, reduction):
    rng = np.random.default_rng(82)
    x = rng.standard_normal((3, 17, 1000)).astype(F32)
    ids = rng.integers(0, 1000, (3, 17)).astype(np.int32)
    got, want, gdx, wdx = run_both(sp, x, ids, reduction, language_model=True)
    check(got, want, gdx[:, :-1], wdx[:, :-1], x[:, :-1], ids[:, 1:].astype(np.int64), reduction,
          F32, f"language model {reduction}")
    assert not gdx[:, -1].any() and not np.signbit(gdx[:, -1]).any(), "last position: +0"


@pytest.mark.parametrize("dtype", [F32, F64])
def test_random_cross_entropy_shapes(sp, dtype):
    """Plain and language-model cross entropy over 16 random shapes each
    (batches of 1 to 6 sequences of 1 to 40 positions, 2 to 20000 classes,
    int32 and int64 targets, every reduction) against the oracle."""
    rng = np.random.default_rng(97 if dtype == F32 else 98)
    for case in range(16):
        batch, sequence = int(rng.integers(1, 7)), int(rng.integers(1, 41))
        classes = int(rng.choice([2, 3, 17, 1000, 4097, 8192, 8193, 20000]))
        reduction = ["none", "sum", "mean"][case % 3]
        x = (rng.standard_normal((batch, sequence, classes)) * 2).astype(dtype)
        t = rng.integers(0, classes, (batch, sequence)).astype(np.int64 if case % 2 else np.int32)
        what = f"case {case}: [{batch}, {sequence}, {classes}] {reduction}"
        got, want, gdx, wdx = run_both(sp, x, t, reduction)
        check(got, want, gdx, wdx, x, t.astype(np.int64), reduction, dtype, what)
        if sequence < 2:
            continue  # a language model needs a next token
        got, want, gdx, wdx = run_both(sp, x, t, reduction, language_model=True)
        check(got, want, gdx[:, :-1], wdx[:, :-1], x[:, :-1], t[:, 1:].astype(np.int64),
              reduction, dtype, what + " language model")
        assert not gdx[:, -1].any() and not np.signbit(gdx[:, -1]).any(), what + " last position"


def test_cross_entropy_undefined_rows(sp):
    """Rows with NaN, +inf or only -inf follow log-softmax's special cases:
    the loss is NaN, -(-log k) or inf as the oracle gives, and the gradient
    of an undefined row is NaN."""
    x = np.array([[0.5, np.nan, 1.0, 2.0],
                  [np.inf, 1.0, np.inf, 0.0],
                  [-np.inf, -np.inf, -np.inf, -np.inf],
                  [1.0, -np.inf, 3.0, 0.5]], F32)
    for t in (np.array([0, 0, 1, 2], np.int64), np.array([1, 1, 3, 1], np.int64)):
        got, want, gdx, wdx = run_both(sp, x, t, "none")
        # NaN and infinity positions exact; finite values (log k) within 2 ulp
        assert np.array_equal(np.isnan(got), np.isnan(want)), f"NaN losses, targets {t}"
        special = ~np.isfinite(want)
        assert np.array_equal(got[special & ~np.isnan(want)], want[special & ~np.isnan(want)])
        assert_ulp(got[np.isfinite(want)], want[np.isfinite(want)], 2, "log k losses")
        assert np.array_equal(np.isnan(gdx), np.isnan(wdx)), "NaN pattern of the gradient"
        finite = ~np.isnan(wdx)
        assert np.allclose(gdx[finite], wdx[finite], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [F32, F64])
def test_cross_entropy_negative_infinity_runs(sp, dtype):
    """Masked logits: long runs of -inf before, between and after finite
    values, so that lanes see only -inf for whole batches (and some rows end
    that way), as the forward's streaming sum must handle."""
    rng = np.random.default_rng(83)
    classes = 32768
    x = (rng.standard_normal((6, classes)) * 2).astype(dtype)
    x[0, : classes // 2] = -np.inf            # masked first half
    x[1, :] = -np.inf
    x[1, classes - 3] = 0.25                  # one live logit at the end
    x[2, 1000:] = -np.inf                     # masked tail
    x[3, ::2] = -np.inf                       # every other logit masked
    x[4, :] = -np.inf
    x[4, 7] = 1.5
    x[4, classes - 1] = 1.5                   # two live logits far apart
    x[5, 4096:28672] = -np.inf                # masked middle
    t = np.array([classes - 1, classes - 3, 5, 1, 7, 100], np.int64)
    got, want, gdx, wdx = run_both(sp, x, t, "none")
    finite = np.isfinite(x).astype(np.float64)
    lp = np.where(finite > 0, closed_lp(np.where(finite > 0, x.astype(np.float64), -1e300)),
                  -np.inf)
    picked = -lp[np.arange(6), t]
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= lp_bound(picked, classes, dtype)), f"losses: {err}"
    assert np.array_equal(np.isnan(gdx), np.isnan(wdx)) and not np.isnan(gdx).any()
    eps = np.finfo(dtype).eps
    bound = np.exp(lp) * (lp_bound(np.where(np.isfinite(lp), lp, 0), classes, dtype) + 4 * eps) \
        + 4 * eps * np.abs(wdx) + np.finfo(dtype).tiny
    assert np.all(np.abs(gdx.astype(np.float64) - wdx) <= bound), "dlogits"


def test_cross_entropy_errors(sp):
    device = sp.Device.hip(0)
    logits = sp.Tensor.from_numpy(np.zeros((2, 3), F32)).to(device)
    ok = sp.Tensor.from_numpy(np.array([0, 2], np.int64)).to(device)
    with pytest.raises(IndexError, match="outside the class range"):
        sp.loss.cross_entropy(logits, sp.Tensor.from_numpy(np.array([0, 3], np.int64)).to(device))
    with pytest.raises(IndexError):
        sp.loss.cross_entropy(logits, sp.Tensor.from_numpy(np.array([-1, 0], np.int32)).to(device))
    with pytest.raises(ValueError, match="Int32 or Int64"):
        sp.loss.cross_entropy(logits, sp.Tensor.from_numpy(np.array([0.0, 1.0], F32)).to(device))
    with pytest.raises(ValueError, match="shape does not match"):
        sp.loss.cross_entropy(logits, sp.Tensor.from_numpy(np.array([0, 1, 2], np.int64)).to(device))
    with pytest.raises(ValueError, match="same Device"):
        sp.loss.cross_entropy(logits, sp.Tensor.from_numpy(np.array([0, 1], np.int64)))
    with pytest.raises(ValueError, match="Float32 or Float64"):
        sp.loss.cross_entropy(ok, ok)
    with pytest.raises(ValueError, match="incompatible shapes"):
        lm = sp.Tensor.from_numpy(np.zeros((2, 1, 3), F32)).to(device)
        sp.loss.language_model_cross_entropy(lm, sp.Tensor.from_numpy(np.zeros((2, 1), np.int64)).to(device))
    assert float(sp.loss.cross_entropy(logits, ok).to(sp.Device.cpu()).numpy()) == pytest.approx(np.log(3))


# ------------------------------------------------ reference-compatible ABI

def test_validate_targets(hip):
    import ctypes

    lib = hip.load()
    for dtype, code in ((np.int32, hip.INT32), (np.int64, hip.INT64)):
        for values, expected in (([0, 4, 2], 0), ([0, 5, 2], 1), ([-1, 0], 1)):
            buffer = hip.DeviceBuffer.from_numpy(np.array(values, dtype))
            flag = ctypes.c_int32(7)
            hip.call("spar_hip_validate_targets", ctypes.byref(flag), buffer.ptr, len(values), 5,
                     code, 0)
            assert flag.value == expected, (values, dtype)
    assert lib.spar_hip_validate_targets(None, None, 0, 5, hip.INT32, 0).code == 1


@pytest.mark.parametrize("language_model", [0, 1])
def test_nll_gather_and_scatter_are_exact(hip, language_model):
    rng = np.random.default_rng(83)
    batch, sequence, classes = 3, 6, 11
    lp = rng.standard_normal((batch * sequence, classes)).astype(F32)
    targets = rng.integers(0, classes, batch * sequence).astype(np.int64)
    if language_model:
        count = batch * (sequence - 1)
        index = np.arange(count)
        rows = (index // (sequence - 1)) * sequence + index % (sequence - 1)
        picked = targets[rows + 1]
    else:
        count = batch * sequence
        rows = np.arange(count)
        picked = targets
    out = hip.DeviceBuffer(count * 4)
    lp_d, t_d = hip.DeviceBuffer.from_numpy(lp), hip.DeviceBuffer.from_numpy(targets)
    hip.call("spar_hip_launch_nll_forward", out.ptr, lp_d.ptr, t_d.ptr, count, classes, sequence,
             hip.FLOAT32, hip.INT64, language_model, 0)
    assert_bitexact(out.to_numpy(F32, (count,)), -lp[rows, picked], "nll forward")
    g = rng.standard_normal(count).astype(F32)
    g_d = hip.DeviceBuffer.from_numpy(g)
    grad = hip.DeviceBuffer(lp.size * 4)
    hip.call("spar_hip_zero", grad.ptr, lp.size * 4, 0)
    hip.call("spar_hip_launch_nll_backward", grad.ptr, g_d.ptr, t_d.ptr, count, classes, sequence,
             hip.FLOAT32, hip.INT64, language_model, 0)
    want = np.zeros_like(lp)
    want[rows, picked] = F32(0) - g
    assert_bitexact(grad.to_numpy(F32, lp.shape), want, "nll backward")
