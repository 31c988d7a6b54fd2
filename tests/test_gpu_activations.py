"""Activation parity (activations_c.c:124-158, activations.asm:352-413).

Piecewise-linear activations (leaky_relu, hardswish, hardtanh) are bit-exact.
Transcendental ones use the same double formula: REL32 (1e-5 relative) for
f32 outputs and REL64 (1e-12 relative + 1e-15 absolute) for f64 outputs,
against the oracle (glibc libm) on inputs normal(0,4) with 1% set to +-30.
"""

import numpy as np
import pytest

from conftest import GPU, rel_close, same_bits

pytestmark = GPU

EXACT = {"leaky_relu", "hardswish", "hardtanh"}
ACTS = ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh", "sigmoid"]
ALPHA = {"leaky_relu": 0.01, "elu": 1.0}


def _inputs(dt, n=1 << 20, seed=4):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 4, n)
    idx = rng.choice(n, size=n // 100, replace=False)
    x[idx] = np.where(rng.random(idx.size) < 0.5, -30.0, 30.0)
    x[:8] = [0.0, -0.0, 3.0, -3.0, 1.0, -1.0, 1e-310, -700.0]
    return x.astype(dt)


def _run(pn, name, x):
    import ctypes
    t = pn.Tensor.from_numpy(x)
    out = pn.Tensor.create(t.shape, t.dtype)
    lib = pn.core._lib
    if name == "sigmoid":
        rc = lib.neural_sigmoid(out._ptr, t._ptr)
    elif name in ALPHA:
        rc = getattr(lib, "act_" + name)(out._ptr, t._ptr, ctypes.c_double(ALPHA[name]))
    else:
        rc = getattr(lib, "act_" + name)(out._ptr, t._ptr)
    assert rc == 0
    return out.numpy()


@pytest.mark.parametrize("name", ACTS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_activation(pn, ora, name, dt):
    x = _inputs(dt)
    got = _run(pn, name, x)
    want = ora.act(name, x, ALPHA.get(name, 0.0))
    if name in EXACT:
        same_bits(got, want)
    elif dt == np.float32:
        rel_close(got, want, 1e-5, 0.0, name)
    else:
        rel_close(got, want, 1e-12, 1e-15, name)


def test_activation_4d_nchw(pn, ora):
    """cfg3 layout [64,64,128,128] at a reduced batch (N=2), NCHW contiguous."""
    x = _inputs(np.float32, n=2 * 64 * 128 * 128, seed=9).reshape(2, 64, 128, 128)
    t = pn.Tensor.from_numpy(x)
    y = pn.GELU()(t).numpy()
    rel_close(y, ora.act("gelu", x.ravel()).reshape(x.shape), 1e-5, 0.0, "gelu 4d")
    y = pn.LeakyReLU(0.2)(t).numpy()
    same_bits(y, ora.act("leaky_relu", x.ravel(), 0.2).reshape(x.shape))


def test_modules_and_aliases(pn, ora):
    x = _inputs(np.float64, n=4096, seed=3)
    t = pn.Tensor.from_numpy(x)
    for mod, name, alias in [(pn.Mish(), "mish", "neural_mish"), (pn.Softplus(), "softplus", "neural_softplus"),
                             (pn.Swish(), "swish", "neural_swish"), (pn.SELU(), "selu", "neural_selu"),
                             (pn.Tanh(), "tanh", "neural_tanh"), (pn.HardSwish(), "hardswish", "neural_hardswish")]:
        want = ora.act(name, x)
        rel_close(mod(t).numpy(), want, 1e-12, 1e-15, name)
        out = pn.Tensor.create(t.shape, t.dtype)
        assert getattr(pn.core._lib, alias)(out._ptr, t._ptr) == 0
        rel_close(out.numpy(), want, 1e-12, 1e-15, alias)
    assert pn.core._lib.act_gelu(None, t._ptr) == pn.NeuralError.NULL_POINTER


@pytest.mark.parametrize("name", ["tanh", "gelu", "mish", "softplus", "swish", "elu", "selu", "sigmoid"])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_activation_dense_sweep(pn, ora, name, dt):
    """Every region of the closed forms: a dense grid over [-40, 40] (the
    cancellation tails of softplus/mish/gelu and the clamps of tanh included),
    the branch points, and the special values."""
    grid = np.linspace(-40.0, 40.0, 2_000_001)
    pts = np.array([0.0, -0.0, 2.0 ** -7, -2.0 ** -7, 22.0, -22.0, 19.06, -19.06, 1e-30, -1e-30, 1e-40, -1e-40,
                    88.7, -88.7, 103.9, -103.9, 709.78, 709.79, -745.2, 1e30, -1e30, 3.4e38, -3.4e38,
                    np.inf, -np.inf, np.nan])
    x = np.concatenate([grid, pts]).astype(dt)
    got = _run(pn, name, x)
    want = ora.act(name, x, ALPHA.get(name, 0.0))
    if dt == np.float32:
        rel_close(got, want, 1e-5, 0.0, name)
    else:
        rel_close(got, want, 1e-12, 1e-15, name)
    z = (want == 0) & ~np.isnan(want)
    assert np.array_equal(np.signbit(got[z]), np.signbit(want[z])), f"{name}: sign of zero differs"


@pytest.mark.parametrize("name,alpha", [("elu", 1.0), ("elu", 0.5), ("elu", 2.5), ("selu", 0.0)])
def test_elu_selu_f32_small_negative(pn, ora, name, alpha):
    """f32 elu / selu take the float expm1 below -2^-26 and the reference's
    double exp(x) - 1.0 above it: a log sweep of negative inputs down to 1e-12
    (where the reference's own cancellation sets the low digits), the points
    around the switch, and the fused bias-add form of the same functors."""
    import ctypes
    t26 = 2.0 ** -26
    x = np.concatenate([-np.logspace(-12, 1, 200_001), np.logspace(-12, 1, 2001),
                        [-t26, -t26 * (1 + 2 ** -23), -t26 * (1 - 2 ** -24), -1.1 * t26, -0.9 * t26,
                         0.0, -0.0, -88.0, -104.0, -np.inf, np.nan]]).astype(np.float32)
    t = pn.Tensor.from_numpy(x)
    out = pn.Tensor.create(t.shape, t.dtype)
    lib = pn.core._lib
    if name == "elu":
        assert lib.act_elu(out._ptr, t._ptr, ctypes.c_double(alpha)) == 0
    else:
        assert lib.act_selu(out._ptr, t._ptr) == 0
    got = out.numpy()
    want = ora.act(name, x, alpha)
    rel_close(got, want, 1e-5, 0.0, name)
    z = (want == 0) & ~np.isnan(want)
    assert np.array_equal(np.signbit(got[z]), np.signbit(want[z]))
    # bias add + activation: x + 0 rounds to x, so the result is the same
    x2 = x[: 4096 * 48].reshape(48, 4096) if x.size >= 4096 * 48 else None
    if x2 is not None:
        b = np.zeros(4096, dtype=np.float32)
        tx, tb = pn.Tensor.from_numpy(np.ascontiguousarray(x2)), pn.Tensor.from_numpy(b)
        o2 = pn.Tensor.create(tx.shape, tx.dtype)
        code = 6 if name == "elu" else 7  # NEURAL_ACT_ELU / NEURAL_ACT_SELU (neural_api.h)
        assert lib.neural_bias_add_act(o2._ptr, tx._ptr, tb._ptr, code, ctypes.c_double(alpha)) == 0
        rel_close(o2.numpy(), want[: x2.size].reshape(x2.shape), 1e-5, 0.0, name + " fused")


# ---- cfg3 at its full size ------------------------------------------------------------------

CFG3_SHAPE = (64, 64, 128, 128)
WIN = 1 << 19


def test_gelu_f32_every_float_around_tail_threshold(pn, ora):
    """Every float x whose GELU argument z = sqrt(2/pi)(x + 0.044715 x^3) lies
    in [-11, -7] (x in [-5.75, -4.55], about 2.5 M values): the float head
    above z = -8 and the double tail below it both within REL32 of the
    reference formula (activations_c.c:124-131) evaluated by the oracle."""
    lo = np.float32(4.55).view(np.uint32)
    hi = np.float32(5.75).view(np.uint32)
    x = (np.arange(lo, hi + 1, dtype=np.uint32) | np.uint32(0x80000000)).view(np.float32)
    got = _run(pn, "gelu", x)
    want = ora.act("gelu", x, 0.0)
    rel_close(got, want, 1e-5, 0.0, "gelu f32 around z = -8")
    z = np.sqrt(2.0 / np.pi) * (x.astype(np.float64) + 0.044715 * x.astype(np.float64) ** 3)
    assert z.min() < -11.0 and z.max() > -7.0


def _torch_formula(torch, name, x):
    """The reference's double formula (activations_c.c:124-158) in torch
    float64, the operation order kept; used as the full-tensor check of the
    f32 outputs (REL32), whose 1e-5 bar is far above libm's last-ulp
    differences."""
    if name == "tanh":
        return torch.tanh(x)
    if name == "gelu":
        return 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)))
    if name == "leaky_relu":
        return torch.where(x >= 0, x, 0.01 * x)
    if name == "elu":
        return torch.where(x > 0, x, 1.0 * (torch.exp(x) - 1.0))
    if name == "selu":
        lam, alp = 1.0507009873554804934193349852946, 1.6732632423543772848170429916717
        return torch.where(x > 0, lam * x, lam * alp * (torch.exp(x) - 1.0))
    if name == "swish":
        return x / (1.0 + torch.exp(-x))
    if name == "mish":
        return x * torch.tanh(torch.log(1.0 + torch.exp(x)))
    if name == "hardswish":
        return torch.where(x <= -3.0, torch.zeros_like(x), torch.where(x >= 3.0, x, x * (x + 3.0) / 6.0))
    if name == "softplus":
        return torch.log(1.0 + torch.exp(x))
    if name == "hardtanh":
        return torch.clamp(x, -1.0, 1.0)
    raise ValueError(name)


@pytest.fixture(scope="module")
def cfg3_input():
    """BASELINE cfg3: N(0,4) over [64,64,128,128] in double, 1% of the
    elements (chosen without replacement) set to +-30."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    x = torch.randn(*CFG3_SHAPE, device="cuda", generator=g, dtype=torch.float64) * 4
    n = x.numel()
    sat = torch.randperm(n, device="cuda", generator=g)[: n // 100]
    x.view(-1)[sat] = 30.0 * (torch.randint(0, 2, (sat.numel(),), device="cuda", generator=g).double() * 2 - 1)
    torch.cuda.synchronize()
    yield x
    del x, sat
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dt_name", ["f32", "f64"])
def test_activations_cfg3_full_size(pn, ora, cfg3_input, dt_name):
    """All ten activations on the full cfg3 tensor (67,108,864 elements,
    NCHW contiguous).  Windows of 2^19 elements at the start, the middle and
    the end against the oracle (glibc libm, the reference's formulas):
    piecewise bit-exact, f32 REL32, f64 REL64.  f32 outputs are also checked
    over the whole tensor against the double formula evaluated by torch."""
    import ctypes
    import torch
    lib = pn.core._lib
    dt = torch.float32 if dt_name == "f32" else torch.float64
    x = cfg3_input.to(dt).contiguous()
    y = torch.empty_like(x)
    tx, ty = pn.Tensor.from_torch(x), pn.Tensor.from_torch(y)
    n = x.numel()
    starts = [0, n // 2 - WIN // 2 + 3, n - WIN]
    xf = x.view(-1)
    xwin = [xf[s:s + WIN].cpu().numpy() for s in starts]
    assert sum(int((np.abs(w) == 30.0).sum()) for w in xwin) > 10000
    x64 = x.double() if dt_name == "f32" else None
    for name in ["tanh", "gelu", "leaky_relu", "elu", "selu", "swish", "mish", "hardswish", "softplus", "hardtanh"]:
        fn = getattr(lib, "act_" + name)
        rc = fn(ty._ptr, tx._ptr, ctypes.c_double(ALPHA[name])) if name in ALPHA else fn(ty._ptr, tx._ptr)
        assert rc == 0, name
        torch.cuda.synchronize()
        yf = y.view(-1)
        for s, xw in zip(starts, xwin):
            got = yf[s:s + WIN].cpu().numpy()
            want = ora.act(name, xw, ALPHA.get(name, 0.0))
            if name in EXACT:
                same_bits(got, want)
            elif dt_name == "f32":
                rel_close(got, want, 1e-5, 0.0, f"{name} window {s}")
            else:
                rel_close(got, want, 1e-12, 1e-15, f"{name} window {s}")
        if dt_name == "f32":
            ref = _torch_formula(torch, name, x64).float()
            if name in EXACT:
                assert torch.equal(y, ref), name
            else:
                yd = y.double()
                rd = ref.double()
                fin = torch.isfinite(rd)
                assert torch.equal(torch.isnan(yd), torch.isnan(rd)), name
                assert torch.equal(yd[~fin & ~torch.isnan(rd)], rd[~fin & ~torch.isnan(rd)]), name
                err = (yd[fin] - rd[fin]).abs() - 1e-5 * rd[fin].abs()
                assert float(err.max()) <= 0.0, (name, float(err.max()))
                del yd, rd, fin, err
            del ref
    del x, y, x64
