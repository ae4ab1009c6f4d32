#!/usr/bin/env python3
"""Write the golden vectors that pin the oracle's END-TO-END COMPOSITION.

What this pins that nothing else can: stage order, skip placement (added before the
up-conv), W/SW alternation starting unshifted in every stage including the up stages,
conv-half-first concatenation, the conv-half residual, pre-norm blocks. Those are
properties of the reference's network walk, not of any single op, so they are taken
from the reference's own numpy transcription, ``tools/reference.py`` (jacobsparts/
scunet-rs, reference.py:165-349), run HERE, in the build container, on this build's
seeded synthetic checkpoint. The reference does not travel: only the resulting arrays
(inputs and expected outputs) are committed, as ``golden.npz``.

Vectors written (all float32):
  fwd64_in / fwd64_out        config-1 style 64x64 colour input and SCUNet.forward output
  fwd80x72_in / fwd80x72_out  an 80x72 input that pads on both axes (to 128x128)
  stage64_<name>_val          a fixed sparse sample (indices: sample_idx(n, 2048, 1000+i)) of
                              each of the 16 stage planes at 64x64, computed with the
                              reference's own stage/conv primitives
  stage64_<name>_stats        [max|x|, mean, sqrt(mean x^2)] of the full plane
  blk_<k>_out                 conv_trans_block(x, prefix, shifted) on small planes; the input
                              is synth.seq(c*h*w, 0.53 + 0.01k) (its float64 sum: blk_<k>_insum)
  wmsa_<k>_out                wmsa(layer_norm(x)) on a token plane (attention alone); input
                              synth.seq(h*w*t, 0.43 + 0.01k) (wmsa_<k>_insum)
  weights_check               sums of a few tensors, to detect a different checkpoint

Run: python tests/golden/make_golden.py  (needs /root/reference; takes ~1 min)
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(HERE, "..", ".."))
sys.path.insert(0, os.path.join(REPO, "scunet-rs_amd"))
from scunet_hip import synth  # noqa: E402

REF = "/root/reference/tools/reference.py"

STAGES = ["m_head", "m_down1_blocks", "m_down1", "m_down2_blocks", "m_down2", "m_down3_blocks",
          "m_down3", "m_body", "m_up3_up", "m_up3", "m_up2_up", "m_up2", "m_up1_up", "m_up1",
          "m_tail_in", "m_tail"]

BLOCK_CASES = [
    # (prefix, h, w, shifted)
    ("m_down1.0", 16, 16, False),
    ("m_down1.1", 16, 16, True),
    ("m_down2.1", 16, 24, True),
    ("m_body.0", 8, 16, False),
    ("m_body.1", 8, 8, True),
    ("m_up1.2", 24, 16, True),
]

WMSA_CASES = [
    # (prefix, h, w, shifted)
    ("m_down1.0", 16, 16, False),
    ("m_down1.1", 16, 24, True),
    ("m_body.1", 16, 16, True),
]


def weights_check(t):
    names = ["m_head.0.weight", "m_down1.0.trans_block.msa.relative_position_params",
             "m_body.3.trans_block.mlp.2.bias", "m_up1.4.conv_block.2.weight", "m_tail.0.weight"]
    return np.array([float(np.asarray(t[n], np.float64).sum()) for n in names], np.float64)


def sample_idx(n, k, seed):
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n, size=min(k, n), replace=False)).astype(np.int64)


def main():
    spec = importlib.util.spec_from_file_location("scunet_reference_py", REF)
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)

    wpath = synth.weights_file(seed=0)
    w, meta = ref.read_safetensors(wpath)
    model = ref.SCUNet(w, meta)
    out = {"weights_check": weights_check(w)}

    # End to end through the reference's own forward (pad, walk, crop).
    x64 = synth.config_input(1)
    out["fwd64_in"] = x64
    out["fwd64_out"] = model.forward(x64[None])[0].astype(np.float32)
    x80 = synth.noisy_image(7, 3, 80, 72, 25)
    out["fwd80x72_in"] = x80
    out["fwd80x72_out"] = model.forward(x80[None])[0].astype(np.float32)

    # The 16 stage planes at 64x64, through the reference's primitives in the order of
    # its forward (reference.py:312-335); the tail output must equal fwd64_out.
    cfg = model.config
    x = x64[None]
    st = {}
    x1 = ref.conv2d(x, w["m_head.0.weight"], pad=1)
    st["m_head"] = x1
    cur = x1
    skips = []
    for k, name in enumerate(["down1", "down2", "down3"]):
        blocks = model.stage(cur, name, cfg[k], False)
        st[f"m_{name}_blocks"] = blocks
        cur = ref.conv2d(blocks, w[f"m_{name}.{cfg[k]}.weight"], stride=2)
        st[f"m_{name}"] = cur
        skips.append(cur)
    cur = model.stage(cur, "body", cfg[3], False)
    st["m_body"] = cur
    for k, name in enumerate(["up3", "up2", "up1"]):
        cur = ref.conv_transpose2x2(cur + skips[2 - k], w[f"m_{name}.0.weight"])
        st[f"m_{name}_up"] = cur
        cur = model._up_blocks(cur, name, cfg[4 + k])
        st[f"m_{name}"] = cur
    cur = cur + x1
    st["m_tail_in"] = cur
    st["m_tail"] = ref.conv2d(cur, w["m_tail.0.weight"], pad=1)
    d = float(np.abs(st["m_tail"][0] - out["fwd64_out"]).max())
    assert d == 0.0, f"stage walk disagrees with SCUNet.forward by {d}"
    for i, name in enumerate(STAGES):
        plane = np.asarray(st[name][0], np.float32).ravel()
        idx = sample_idx(plane.size, 2048, 1000 + i)
        out[f"stage64_{name}_val"] = plane[idx]
        out[f"stage64_{name}_stats"] = np.array(
            [np.abs(plane).max(), plane.mean(), np.sqrt((plane.astype(np.float64) ** 2).mean())],
            np.float64)

    # Blocks and attention alone.
    for k, (prefix, h, wd, shifted) in enumerate(BLOCK_CASES):
        c = w[f"{prefix}.conv1_1.weight"].shape[0]
        xb = synth.seq(c * h * wd, 0.53 + 0.01 * k).reshape(1, c, h, wd)
        out[f"blk_{k}_insum"] = np.array([xb.astype(np.float64).sum()])
        out[f"blk_{k}_out"] = model.conv_trans_block(xb, prefix, shifted)[0].astype(np.float32)
    for k, (prefix, h, wd, shifted) in enumerate(WMSA_CASES):
        t = w[f"{prefix}.trans_block.msa.linear.weight"].shape[0]
        xt = synth.seq(h * wd * t, 0.43 + 0.01 * k).reshape(1, h, wd, t)
        tp = prefix + ".trans_block"
        ln = ref.layer_norm(xt, w[tp + ".ln1.weight"], w[tp + ".ln1.bias"])
        out[f"wmsa_{k}_insum"] = np.array([xt.astype(np.float64).sum()])
        out[f"wmsa_{k}_out"] = model.wmsa(ln, tp + ".msa", shifted)[0].astype(np.float32)

    dst = os.path.join(HERE, "golden.npz")
    np.savez_compressed(dst, **{k: np.asarray(v) for k, v in out.items()})
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
