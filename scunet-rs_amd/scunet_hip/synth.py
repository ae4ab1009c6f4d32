"""Seeded synthetic SCUNet checkpoints and inputs.

There is no network and no published checkpoint on these machines, so every
weight file used by the tests and the benchmark is generated here from a seed.
The tensor names, shapes and ``__metadata__`` keys are the ones the reference's
loader validates (src/weights.rs:117 for the keys, 204-280 for the shapes) and
that tools/convert.py:227-236 writes, so a file made here loads in the
reference unchanged.

Initialisation (the recipe is also written into the file's metadata):

* Linear weights (qkv, proj, mlp.0, mlp.2): truncated normal, std 0.02,
  values outside +-2 std are redrawn.
* Relative-position tables: the same truncated normal, drawn in upstream's
  pre-view storage ``[(2w-1)^2][heads]`` and re-laid to ``[heads][2w-1][2w-1]``
  exactly as network_scunet.py:42-47 does (view, transpose(1,2), transpose(0,1)).
* Convolution weights (3x3, 1x1, 2x2 and the transposed 2x2): Kaiming-uniform as
  torch's default, bound 1/sqrt(fan_in) with fan_in = shape[1]*kh*kw.
* Biases (conv1_1, conv1_2 and every Linear): uniform +-1/sqrt(fan_in).
* LayerNorm: gamma = 1, beta = 0, or, with ``ln_affine="random"``,
  gamma = 1 + 0.1 N(0,1) and beta = 0.1 N(0,1) so affine indexing is exercised.

Everything is drawn from ``numpy.random.default_rng(seed)`` (PCG64) in the
order of :func:`tensor_specs`, so a seed names one file on any machine.
"""
import hashlib
import os

import numpy as np

from .safetensors_io import write_safetensors

STAGES = ("down1", "down2", "down3", "body", "up3", "up2", "up1")
# Block width multiplier of each stage relative to dim (c = dim * mult).
STAGE_MULT = {"down1": 1, "down2": 2, "down3": 4, "body": 8, "up3": 4, "up2": 2, "up1": 1}
# Downsampling steps of each stage's plane.
STAGE_LEVEL = {"down1": 0, "down2": 1, "down3": 2, "body": 3, "up3": 2, "up2": 1, "up1": 0}


def tensor_specs(in_nc=3, dim=64, config=(4, 4, 4, 4, 4, 4, 4), head_dim=32, window=8):
    """``[(name, shape, kind)]`` in the order src/weights.rs:204-263 lists them.

    ``kind`` is one of conv, convT, conv_bias, linear, linear_bias, ln_w, ln_b, relpos.
    """
    span = 2 * window - 1
    specs = [("m_head.0.weight", (dim, in_nc, 3, 3), "conv"),
             ("m_tail.0.weight", (in_nc, dim, 3, 3), "conv")]
    for si, name in enumerate(STAGES):
        count = config[si]
        c = dim * STAGE_MULT[name]
        t = c // 2
        first = 1 if name.startswith("up") else 0
        if first:
            specs.append((f"m_{name}.0.weight", (2 * c, c, 2, 2), "convT"))
        for b in range(first, first + count):
            p = f"m_{name}.{b}"
            specs += [
                (f"{p}.conv1_1.weight", (c, c, 1, 1), "conv"),
                (f"{p}.conv1_1.bias", (c,), "conv_bias"),
                (f"{p}.conv1_2.weight", (c, c, 1, 1), "conv"),
                (f"{p}.conv1_2.bias", (c,), "conv_bias"),
                (f"{p}.conv_block.0.weight", (t, t, 3, 3), "conv"),
                (f"{p}.conv_block.2.weight", (t, t, 3, 3), "conv"),
                (f"{p}.trans_block.ln1.weight", (t,), "ln_w"),
                (f"{p}.trans_block.ln1.bias", (t,), "ln_b"),
                (f"{p}.trans_block.ln2.weight", (t,), "ln_w"),
                (f"{p}.trans_block.ln2.bias", (t,), "ln_b"),
                (f"{p}.trans_block.mlp.0.weight", (4 * t, t), "linear"),
                (f"{p}.trans_block.mlp.0.bias", (4 * t,), "linear_bias"),
                (f"{p}.trans_block.mlp.2.weight", (t, 4 * t), "linear"),
                (f"{p}.trans_block.mlp.2.bias", (t,), "linear_bias"),
                (f"{p}.trans_block.msa.embedding_layer.weight", (3 * t, t), "linear"),
                (f"{p}.trans_block.msa.embedding_layer.bias", (3 * t,), "linear_bias"),
                (f"{p}.trans_block.msa.linear.weight", (t, t), "linear"),
                (f"{p}.trans_block.msa.linear.bias", (t,), "linear_bias"),
                (f"{p}.trans_block.msa.relative_position_params",
                 (t // head_dim, span, span), "relpos"),
            ]
        if name.startswith("down"):
            specs.append((f"m_{name}.{count}.weight", (2 * c, c, 2, 2), "conv"))
    return specs


def _trunc_normal(rng, shape, std):
    a = rng.standard_normal(size=shape) * std
    bad = np.abs(a) > 2 * std
    while bad.any():
        a[bad] = rng.standard_normal(size=int(bad.sum())) * std
        bad = np.abs(a) > 2 * std
    return a


def make_weights(seed=0, in_nc=3, dim=64, config=(4, 4, 4, 4, 4, 4, 4), head_dim=32,
                 window=8, ln_affine="identity"):
    """``({name: float32 array}, metadata)`` for a seeded random-init SCUNet."""
    rng = np.random.default_rng(seed)
    out = {}
    # The biases' fan_in is the layer's input width; remember it per prefix.
    for name, shape, kind in tensor_specs(in_nc, dim, config, head_dim, window):
        if kind in ("conv", "convT"):
            fan_in = shape[1] * shape[2] * shape[3]
            bound = 1.0 / np.sqrt(fan_in)
            a = rng.uniform(-bound, bound, size=shape)
        elif kind == "conv_bias":
            bound = 1.0 / np.sqrt(shape[0])
            a = rng.uniform(-bound, bound, size=shape)
        elif kind == "linear":
            a = _trunc_normal(rng, shape, 0.02)
        elif kind == "linear_bias":
            wname = name[: -len("bias")] + "weight"
            fan_in = [s for n, s, _ in _SPEC_CACHE(in_nc, dim, config, head_dim, window)
                      if n == wname][0][1]
            bound = 1.0 / np.sqrt(fan_in)
            a = rng.uniform(-bound, bound, size=shape)
        elif kind == "ln_w":
            a = np.ones(shape) if ln_affine == "identity" else 1.0 + 0.1 * rng.standard_normal(shape)
        elif kind == "ln_b":
            a = np.zeros(shape) if ln_affine == "identity" else 0.1 * rng.standard_normal(shape)
        elif kind == "relpos":
            heads, span, _ = shape
            raw = _trunc_normal(rng, (span * span, heads), 0.02)
            a = raw.reshape(span, span, heads).transpose(0, 2, 1).transpose(1, 0, 2)
        else:
            raise AssertionError(kind)
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
    variant = "color-real-psnr" if in_nc == 3 else "gray-25"
    meta = {
        "arch": "scunet",
        "variant": variant,
        "in_nc": in_nc,
        "dim": dim,
        "config": ",".join(str(v) for v in config),
        "head_dim": head_dim,
        "window_size": window,
        "synthetic_seed": seed,
        "synthetic_init": ("linear trunc_normal(0.02, redraw beyond 2std); relpos same, "
                           "[(2w-1)^2][heads] re-laid to [heads][2w-1][2w-1]; conv kaiming_uniform "
                           "bound 1/sqrt(fan_in); biases U(+-1/sqrt(fan_in)); ln " + ln_affine),
    }
    return out, meta


_spec_memo = {}


def _SPEC_CACHE(*key):
    if key not in _spec_memo:
        _spec_memo[key] = tensor_specs(*key)
    return _spec_memo[key]


def default_cache_dir():
    d = os.environ.get("SCUNET_WEIGHTS_DIR")
    if d:
        return d
    here = os.path.dirname(os.path.abspath(__file__))
    return os.path.join(here, "..", "..", "_build", "weights")


def weights_file(seed=0, in_nc=3, ln_affine="identity", directory=None, **kw):
    """Path of the seeded checkpoint, generating it on first use (~72 MB for colour)."""
    directory = directory or default_cache_dir()
    os.makedirs(directory, exist_ok=True)
    tag = hashlib.sha1(repr((seed, in_nc, ln_affine, sorted(kw.items()))).encode()).hexdigest()[:8]
    path = os.path.join(directory, f"scunet-synth-in{in_nc}-s{seed}-{ln_affine}-{tag}.safetensors")
    if not os.path.exists(path):
        tensors, meta = make_weights(seed=seed, in_nc=in_nc, ln_affine=ln_affine, **kw)
        tmp = path + f".tmp{os.getpid()}"
        write_safetensors(tmp, tensors, meta)
        os.replace(tmp, path)
    return path


# ---------------------------------------------------------------------------
# Inputs (benchmark configs 1-5)
# ---------------------------------------------------------------------------

def _clamp01(x):
    return np.clip(x, 0.0, 1.0).astype(np.float32)


def uniform_texture(rng, c, h, w):
    return rng.random((c, h, w))


def gradient_texture(rng, c, h, w):
    """Smooth random gradients plus uniform[0,1] high-frequency patches."""
    yy, xx = np.meshgrid(np.linspace(0, 1, h), np.linspace(0, 1, w), indexing="ij")
    img = np.empty((c, h, w))
    for ch in range(c):
        a, b, d = rng.uniform(-1, 1, 3)
        f1, f2 = rng.uniform(0.5, 3.0, 2)
        ph1, ph2 = rng.uniform(0, 2 * np.pi, 2)
        img[ch] = (0.5 + 0.25 * (a * yy + b * xx) + 0.15 * d
                   + 0.1 * np.sin(2 * np.pi * f1 * yy + ph1) * np.cos(2 * np.pi * f2 * xx + ph2))
    n_patch = max(1, (h * w) // 4096)
    for _ in range(n_patch):
        ph = int(rng.integers(4, max(5, h // 8)))
        pw = int(rng.integers(4, max(5, w // 8)))
        y0 = int(rng.integers(0, max(1, h - ph)))
        x0 = int(rng.integers(0, max(1, w - pw)))
        img[:, y0:y0 + ph, x0:x0 + pw] = rng.random((c, ph, pw))
    return img


def noisy_image(seed, c, h, w, sigma255, texture="uniform"):
    """``[c][h][w]`` float32: texture + N(0, (sigma/255)^2), clamped to [0, 1]."""
    rng = np.random.default_rng(seed)
    tex = uniform_texture(rng, c, h, w) if texture == "uniform" else gradient_texture(rng, c, h, w)
    noise = rng.standard_normal((c, h, w)) * (sigma255 / 255.0)
    return _clamp01(tex + noise)


CONFIGS = {
    1: dict(c=3, h=64, w=64, sigma255=25, texture="uniform", seed=101),
    2: dict(c=3, h=512, w=512, sigma255=50, texture="gradient", seed=102),
    3: dict(c=3, h=1080, w=1920, sigma255=15, texture="gradient", seed=103),
    4: dict(c=1, h=4096, w=4096, sigma255=25, texture="uniform", seed=104),
}


def config_input(k):
    cfg = CONFIGS[k]
    return noisy_image(cfg["seed"], cfg["c"], cfg["h"], cfg["w"], cfg["sigma255"], cfg["texture"])


def seq(n, a):
    """The reference tests' deterministic sequence sin(sin(i*a)*0.7 + 0.3a) (tests/cuda_ops.rs:36-38)."""
    i = np.arange(n, dtype=np.float32)
    return np.sin(np.sin(i * np.float32(a)) * np.float32(0.7) + np.float32(0.3) * np.float32(a)).astype(np.float32)
