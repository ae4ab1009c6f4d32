"""The default fp32 mode's split-operand products against float64 and against the fp32 MFMA.

In SCUNET_HIP_FP32 (the default) the persistent GEMM (1x1 at 256 / 512 channels, the 2x2
down- and up-convs, the token linears), the resident-weight 1x1 (64 / 128 channels), the
t = 128 / 256 MLP and the window kernels form each fp32 product from an exact three-way bf16
split of both operands (x = h + m + l) as the six part products hh, hm, mh, hl, lh, mm on the
bf16 matrix cores, accumulated in fp32. The dropped ml + lm + ll are below 2^-25 |ab|, so the
result must be as close to the exact (float64) value as the fp32 matrix cores'
(SCUNET_HIP_FP32_MFMA) result is:

* every output within 1e-6 of sum |a b| of its exact value, in both modes (the fp32 bound
  K 2^-24 is far above what random-sign accumulation gives at these K);
* the mean relative error of the split form at most 1.5x that of the fp32 MFMA. A form that
  dropped hl / lh or mm (each up to 2^-17 |ab| per product) would be several times worse;
  inputs span 2^-10 .. 2^10 so that every part is exercised.

The whole forward in both fp32 modes is checked against the oracle stage by stage (1e-4,
the north star's bound) and against each other.
"""
import numpy as np
import pytest

import oracle as O
from conftest import max_abs

pytestmark = pytest.mark.gpu

STAGE_TOL = 1e-4


@pytest.fixture(scope="module")
def be(weights_path):
    from scunet_hip import Hip
    h = Hip(weights_path)
    yield h
    h.close()


def wide(rng, shape):
    """N(0, 1) values scaled by 2^k, k uniform in [-10, 10]: every bf16 part is non-zero."""
    return (rng.standard_normal(shape) * np.exp2(rng.integers(-10, 11, shape))).astype(np.float32)


def rel_err(got, exact, scale):
    return np.abs(got.astype(np.float64) - exact) / scale


def both_modes(be, fn):
    assert be.precision() == "fp32"
    a = fn()
    be.set_precision("fp32_mfma")
    try:
        b = fn()
    finally:
        be.set_precision("fp32")
    return a, b


def check(what, split, mfma, exact, scale):
    e6, em = rel_err(split, exact, scale), rel_err(mfma, exact, scale)
    assert e6.max() <= 1e-6, (what, float(e6.max()))
    assert em.max() <= 1e-6, (what, float(em.max()))
    assert e6.mean() <= 1.5 * em.mean() + 1e-12, (what, float(e6.mean()), float(em.mean()))


def test_precision_modes(be):
    assert be.precision() == "fp32"
    be.set_precision("fp32_mfma")
    assert be.precision() == "fp32_mfma"
    be.set_precision("fp16")
    assert be.precision() == "fp16"
    be.set_precision("fp32")
    assert be.precision() == "fp32"
    with pytest.raises(Exception, match="SCUNET_HIP_FP32_MFMA"):
        be._check(be._lib.scunet_hip_set_precision(be._h, 5))
    assert be.precision() == "fp32"


@pytest.mark.parametrize("name,rows", [("m_body.0.trans_block.mlp.0", 333), ("m_down2.0.trans_block.mlp.0", 257),
                                       ("m_up3.2.trans_block.mlp.2", 130), ("m_body.1.trans_block.msa.linear", 200)])
def test_linear_split_against_float64(be, owt, name, rows):
    wt, b = owt.t[name + ".weight"], owt.t[name + ".bias"]
    co, ci = wt.shape
    x = wide(np.random.default_rng(rows), (rows, ci))
    split, mfma = both_modes(be, lambda: be.linear_probe(name, x, rows, ci, co).reshape(rows, co))
    x64, w64 = x.astype(np.float64), wt.astype(np.float64)
    exact = x64 @ w64.T + b
    scale = np.abs(x64) @ np.abs(w64).T + np.abs(b)
    check(name, split, mfma, exact, scale)


@pytest.mark.parametrize("name,c", [("m_down1.0.conv1_1", 64), ("m_down2.1.conv1_2", 128),
                                    ("m_down3.0.conv1_1", 256), ("m_body.2.conv1_2", 512)])
def test_conv1x1_split_against_float64(be, owt, name, c):
    h, w = 16, 24
    x = wide(np.random.default_rng(c), (c, h, w))
    split, mfma = both_modes(be, lambda: be.op_probe("conv1x1", name, x, c, c, h, w).reshape(c, h * w))
    wt = owt.t[name + ".weight"].reshape(c, c).astype(np.float64)
    b = owt.t[name + ".bias"].astype(np.float64)
    x64 = x.reshape(c, h * w).astype(np.float64)
    exact = wt @ x64 + b[:, None]
    scale = np.abs(wt) @ np.abs(x64) + np.abs(b)[:, None]
    check(name, split, mfma, exact, scale)


def test_stride2_and_transposed_split_against_float64(be, owt):
    h, w = 16, 24
    for name, ci in (("m_down1.4", 64), ("m_down3.4", 256)):
        x = wide(np.random.default_rng(ci), (ci, h, w))
        split, mfma = both_modes(be, lambda: be.op_probe("conv2x2s2", name, x, ci, 2 * ci, h, w))
        wt = owt.t[name + ".weight"].astype(np.float64)                     # [co][ci][2][2]
        p = x.astype(np.float64).reshape(ci, h // 2, 2, w // 2, 2)            # [ci][i][ky][j][kx]
        exact = np.einsum("ocyx,ciyjx->oij", wt, p)
        scale = np.einsum("ocyx,ciyjx->oij", np.abs(wt), np.abs(p))
        check(name, split.reshape(exact.shape), mfma.reshape(exact.shape), exact, scale)
    for name, ci in (("m_up3.0", 512), ("m_up1.0", 128)):
        x = wide(np.random.default_rng(ci + 1), (ci, 8, 16))
        split, mfma = both_modes(be, lambda: be.op_probe("conv_t2x2", name, x, ci, ci // 2, 8, 16))
        wt = owt.t[name + ".weight"].astype(np.float64)                     # [ci][co][2][2]
        x64 = x.astype(np.float64)
        exact = np.einsum("coyx,cij->oiyjx", wt, x64).reshape(ci // 2, 16, 32)
        scale = np.einsum("coyx,cij->oiyjx", np.abs(wt), np.abs(x64)).reshape(ci // 2, 16, 32)
        check(name, split.reshape(exact.shape), mfma.reshape(exact.shape), exact, scale)


def test_both_fp32_modes_every_stage_against_cpu(be, owt, golden):
    x = golden["fwd64_in"]
    _, want = O.forward_dump(owt, x)
    outs = {}
    for mode in ("fp32_mfma", "fp32"):
        be.set_precision(mode)
        got = {}
        outs[mode] = be.forward_dump(x, lambda n, v: got.__setitem__(n, v))
        assert list(got) == list(want)
        for name in want:
            d = max_abs(want[name], got[name])
            assert d <= STAGE_TOL, f"{mode} {name}: {d:.3e}"
    assert be.precision() == "fp32"
    assert max_abs(outs["fp32_mfma"], outs["fp32"]) <= 2e-5


def test_both_fp32_modes_agree_at_512(be, owt):
    from scunet_hip import run
    rng = np.random.default_rng(7)
    x = rng.random((3, 512, 512), dtype=np.float32)
    y6 = run(be, x)
    be.set_precision("fp32_mfma")
    try:
        ym = run(be, x)
    finally:
        be.set_precision("fp32")
    assert np.isfinite(y6).all()
    assert max_abs(ym, y6) <= 2e-5
