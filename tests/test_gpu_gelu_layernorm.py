"""The forward's own LayerNorm prologues and GELU, checked in isolation on the device.

GELU and the two LayerNorms run inside the fused window kernels (the attention half and the
MLP at t = 32 and 64, the attention half and the separate MLP kernel at t = 128 and 256), so
they are reached here through ConvTransBlock probes (Cuda::block_dump, cuda.rs:1153-1167) on
a crafted checkpoint whose blocks make one quantity appear at the block output:

* conv1_1 = conv1_2 = identity with zero bias and the 3x3 weights zero, so the block output is
  x + y with y[:, :t] = x[:, :t] and y[:, t:] = x_t + attention half + MLP (cpu.rs:869-970);
* LN1 (cpu.rs:338-357 ahead of the attention, cpu.rs:791-795): q = k = 0 and a relative-position
  bias of +60 on the diagonal make every token attend to itself only (the other 63 weights are
  e^-60 of it), v = proj = identity and mlp.2 = 0: the trans half of the output is 2 x_t + LN1(x_t);
* LN2 (cpu.rs:800-805): proj = 0, mlp.0 = [I; 0] with bias 10 (GELU is the identity to fp32
  precision on [6, 14]), mlp.2 = [I | 0] with bias -10: the trans half is 2 x_t + LN2(x_t);
* GELU (cpu.rs:293-332): x = 0, proj = 0, mlp.0 = 0 with chosen biases v, mlp.2 picks one hidden
  unit per output channel: the trans half is exactly GELU(v) as the kernel evaluates it (the
  fused kernels read Phi from a cubic table of the A&S function, build_gelu_table).

LayerNorm is compared with its closed form in float64 (two-pass variance, eps 1e-5, random
affine); GELU with the exact 0.5 v (1 + erf(v / sqrt 2)) within the Abramowitz & Stegun 7.1.26
bound the reference's CPU path carries (|erf error| < 1.5e-7) plus fp32 rounding, and with the
oracle's own GELU (the reference's f64 A&S cast to f32) within the table's 1e-7 |v| plus fp32
rounding (and 1e-9 |v| beyond +-6, where the table holds Phi at its ends).
"""
import math

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

# Per level: (t, LN1 block, LN2 block, GELU blocks).
LEVELS = [
    (32, "m_down1.0", "m_down1.1", ["m_up1.1", "m_up1.2", "m_up1.3", "m_up1.4"]),
    (64, "m_down2.0", "m_down2.1", ["m_up2.1", "m_up2.2", "m_up2.3", "m_up2.4"]),
    (128, "m_down3.0", "m_down3.1", ["m_up3.1", "m_up3.2", "m_up3.3", "m_up3.4"]),
    (256, "m_body.0", "m_body.1", ["m_body.2", "m_body.3"]),
]


def gelu_sweep(n):
    """n inputs over [-8, 8] plus special points (0, tiny, the A&S polynomial's knees)."""
    v = np.linspace(-8.0, 8.0, n)
    special = [0.0, 1e-4, -1e-4, 0.5, -0.5, 1.0, -1.0, 3.9, -3.9, 6.0, -6.0, 0.75, -2.25]
    v[:len(special)] = special
    return v.astype(np.float32)


def _base_block(t, rng):
    c = 2 * t
    eye = np.eye(c, dtype=np.float32).reshape(c, c, 1, 1)
    heads = t // 32
    return {
        "conv1_1.weight": eye, "conv1_1.bias": np.zeros(c, np.float32),
        "conv1_2.weight": eye.copy(), "conv1_2.bias": np.zeros(c, np.float32),
        "conv_block.0.weight": np.zeros((t, t, 3, 3), np.float32),
        "conv_block.2.weight": np.zeros((t, t, 3, 3), np.float32),
        "trans_block.ln1.weight": (1 + 0.1 * rng.standard_normal(t)).astype(np.float32),
        "trans_block.ln1.bias": (0.1 * rng.standard_normal(t)).astype(np.float32),
        "trans_block.ln2.weight": (1 + 0.1 * rng.standard_normal(t)).astype(np.float32),
        "trans_block.ln2.bias": (0.1 * rng.standard_normal(t)).astype(np.float32),
        "trans_block.msa.embedding_layer.weight": np.zeros((3 * t, t), np.float32),
        "trans_block.msa.embedding_layer.bias": np.zeros(3 * t, np.float32),
        "trans_block.msa.linear.weight": np.zeros((t, t), np.float32),
        "trans_block.msa.linear.bias": np.zeros(t, np.float32),
        "trans_block.msa.relative_position_params": np.zeros((heads, 15, 15), np.float32),
        "trans_block.mlp.0.weight": np.zeros((4 * t, t), np.float32),
        "trans_block.mlp.0.bias": np.zeros(4 * t, np.float32),
        "trans_block.mlp.2.weight": np.zeros((t, 4 * t), np.float32),
        "trans_block.mlp.2.bias": np.zeros(t, np.float32),
    }


@pytest.fixture(scope="module")
def crafted(tmp_path_factory):
    """A checkpoint (the seeded one with the probe blocks replaced) and the GELU inputs."""
    from scunet_hip import synth
    from scunet_hip.safetensors_io import write_safetensors
    tensors, meta = synth.make_weights(seed=0)
    rng = np.random.default_rng(9)
    gelu_in = {}
    for t, ln1, ln2, gelus in LEVELS:
        blk = _base_block(t, rng)
        blk["trans_block.msa.embedding_layer.weight"][2 * t:] = np.eye(t, dtype=np.float32)   # v = x
        blk["trans_block.msa.relative_position_params"][:, 7, 7] = 60.0                      # self only
        blk["trans_block.msa.linear.weight"] = np.eye(t, dtype=np.float32)
        for k, v in blk.items():
            tensors[f"{ln1}.{k}"] = v
        blk = _base_block(t, rng)
        blk["trans_block.mlp.0.weight"][:t] = np.eye(t, dtype=np.float32)
        blk["trans_block.mlp.0.bias"][:t] = 10.0
        blk["trans_block.mlp.0.bias"][t:] = -10.0
        blk["trans_block.mlp.2.weight"][:, :t] = np.eye(t, dtype=np.float32)
        blk["trans_block.mlp.2.bias"][:] = -10.0
        for k, v in blk.items():
            tensors[f"{ln2}.{k}"] = v
        v = gelu_sweep(4 * t)
        for sel, prefix in enumerate(gelus):
            blk = _base_block(t, rng)
            blk["trans_block.ln2.weight"][:] = 1.0
            blk["trans_block.ln2.bias"][:] = 0.0
            blk["trans_block.mlp.0.bias"] = v.copy()
            w2 = np.zeros((t, 4 * t), np.float32)
            w2[np.arange(t), np.arange(t) + sel * t] = 1.0                                 # out o <- hidden o + sel t
            blk["trans_block.mlp.2.weight"] = w2
            for k, val in blk.items():
                tensors[f"{prefix}.{k}"] = val
            gelu_in[prefix] = v[sel * t:(sel + 1) * t]
    path = str(tmp_path_factory.mktemp("crafted") / "crafted.safetensors")
    write_safetensors(path, tensors, meta)
    return path, tensors, gelu_in


def _ln_closed_form(x, g, b):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + 1e-5) * g.astype(np.float64) + b.astype(np.float64)


@pytest.mark.parametrize("t,ln1,ln2,gelus", LEVELS)
def test_layer_norm_prologues_closed_form(crafted, t, ln1, ln2, gelus):
    from scunet_hip import Hip
    path, tensors, _ = crafted
    h, w = 16, 24
    c = 2 * t
    rng = np.random.default_rng(t)
    x = (0.1 * rng.standard_normal((c, h, w)) + 0.05).astype(np.float32)
    xt = x[t:].reshape(t, h * w).T.astype(np.float64)                # [P][t] tokens
    with Hip(path) as be:
        for prefix, which in ((ln1, "ln1"), (ln2, "ln2")):
            want = _ln_closed_form(xt, tensors[f"{prefix}.trans_block.{which}.weight"],
                                   tensors[f"{prefix}.trans_block.{which}.bias"])
            for shift in (0, 4):
                out = be.block_dump(prefix, h, w, shift, x)
                got = out[t:].reshape(t, h * w).T.astype(np.float64) - 2.0 * xt
                d = float(np.abs(got - want).max())
                # fp32 LayerNorm (|values| < 5) plus the roundings of the exposing adds
                # (ulp(14) / 2 for LN2's +-10 and ulp of 2 x_t + LN).
                assert d <= 3e-6, (prefix, which, shift, d)
                assert np.array_equal(out[:t], 2.0 * x[:t]), prefix              # conv half: x + x


@pytest.mark.parametrize("t,ln1,ln2,gelus", LEVELS)
def test_gelu_against_erf(crafted, t, ln1, ln2, gelus):
    from scunet_hip import Hip
    path, _, gelu_in = crafted
    h, w = 16, 16
    c = 2 * t
    x = np.zeros((c, h, w), np.float32)
    with Hip(path) as be:
        for prefix in gelus:
            v = gelu_in[prefix]
            out = be.block_dump(prefix, h, w, 4, x)
            got = out[t:].reshape(t, h * w)
            # every pixel of the plane gives the same t values
            assert np.array_equal(got, np.repeat(got[:, :1], h * w, axis=1)), prefix
            g = got[:, 0].astype(np.float64)
            exact = np.array([0.5 * float(a) * (1.0 + math.erf(float(a) / math.sqrt(2.0))) for a in v])
            # The kernels evaluate v Phi(v) from a cubic table of the A&S Phi (build_gelu_table):
            # the fit and its fp32 evaluation hold Phi to 1e-7 (1e-7 |v| on GELU, plus rounding
            # of the result), and beyond +-6 the table gives v Phi(+-6), Phi(-6) being ~1e-9.
            av = np.abs(v.astype(np.float64))
            ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
            table = 1e-7 * av + 4.0 * ulp + 1e-9 * np.maximum(1.0, av)
            bound = 0.5 * av * 1.5e-7 + table
            assert (np.abs(g - exact) <= bound).all(), (prefix, float(np.abs(g - exact).max()))
            ref = O.gelu(v).astype(np.float64)                 # cpu.rs's A&S in f64, cast to f32
            assert (np.abs(g - ref) <= table).all(), (prefix, float(np.abs(g - ref).max()))
            assert np.array_equal(out[:t], np.zeros((t, h, w), np.float32))
