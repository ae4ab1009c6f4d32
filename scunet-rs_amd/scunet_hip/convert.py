"""Convert a published SCUNet ``.pth`` checkpoint into the safetensors file this backend
(and the reference crate) loads.

    python -m scunet_hip.convert scunet_color_real_psnr.pth scunet-color-real-psnr.safetensors

The output follows tools/convert.py:126-268 of the reference: every tensor of the state
dict in C order (the saved ``relative_position_params`` are a transposed view of
upstream's ``[(2w-1)^2][heads]`` storage, network_scunet.py:42-47, so the copy must
follow the strides, not the storage), tensors sorted by name, and the ``__metadata__``
keys src/weights.rs:117 validates: format, arch, variant, in_nc, dim, config, head_dim,
window_size. ``config`` and ``in_nc`` are read off the tensors (the ConvTransBlock count
of each stage; m_head's input channels), the variant off the file name unless given.

The checkpoint is read with ``torch.load(..., weights_only=True)``, which restores
tensors and plain containers and executes nothing else from the file. Tensors are
written as F32 (this backend's loader reads F32 only).
"""
import argparse
import os
import re
import sys

import numpy as np

from .safetensors_io import write_safetensors

# The eight published checkpoints (file stem -> (in_nc, variant)); all are dim 64,
# config [4,4,4,4,4,4,4].
KNOWN = {
    "scunet_gray_15": (1, "gray-15"),
    "scunet_gray_25": (1, "gray-25"),
    "scunet_gray_50": (1, "gray-50"),
    "scunet_color_15": (3, "color-15"),
    "scunet_color_25": (3, "color-25"),
    "scunet_color_50": (3, "color-50"),
    "scunet_color_real_psnr": (3, "color-real-psnr"),
    "scunet_color_real_gan": (3, "color-real-gan"),
}
STAGES = ("down1", "down2", "down3", "body", "up3", "up2", "up1")

__all__ = ["KNOWN", "load_state_dict", "arch_of", "convert", "main"]


def load_state_dict(path):
    """``{name: float32 C-order ndarray}`` from a torch checkpoint (weights only)."""
    import torch
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(obj, dict) and len(obj) == 1:
        inner = next(iter(obj.values()))
        if isinstance(inner, dict) and any(torch.is_tensor(v) for v in inner.values()):
            obj = inner      # {"params": state_dict} wrappers
    if not isinstance(obj, dict):
        raise ValueError(f"{path}: the checkpoint is not a state dict")
    out = {}
    for k, v in obj.items():
        if torch.is_tensor(v):
            # .contiguous() walks the saved strides (the transposed rel-pos views).
            out[str(k)] = v.detach().to(torch.float32).contiguous().numpy().copy()
    if "m_head.0.weight" not in out:
        raise ValueError(f"{path}: no m_head.0.weight - not an SCUNet checkpoint?")
    return out


def arch_of(state):
    """(in_nc, dim, config) read off the tensors (tools/convert.py:146-170): a stage's
    block count is its largest ConvTransBlock index + 1, minus the up stages' leading
    transposed conv at index 0."""
    def blocks(stage):
        first = 1 if stage.startswith("up") else 0
        idx = [int(k.split(".")[1]) for k in state
               if k.startswith(f"m_{stage}.") and "trans_block" in k and k.split(".")[1].isdigit()]
        return (max(idx) + 1 - first) if idx else 0
    head = state["m_head.0.weight"].shape
    return int(head[1]), int(head[0]), [blocks(s) for s in STAGES]


def convert(src, dst, variant=None, head_dim=32, window=8):
    """Write ``dst``; returns (the metadata written, the number of tensors)."""
    state = load_state_dict(src)
    in_nc, dim, cfg = arch_of(state)
    if in_nc not in (1, 3):
        raise ValueError(f"{src}: m_head has {in_nc} input channels; SCUNet is 1 or 3")
    if variant is None:
        stem = re.sub(r"\.pth$", "", os.path.basename(src))
        kc, variant = KNOWN.get(stem, (in_nc, f"in{in_nc}-unknown"))
        if kc != in_nc:
            print(f"warning: {stem} is published with in_nc={kc}, the weights have {in_nc}", file=sys.stderr)
    if cfg != [4] * 7:
        print(f"warning: the weights are config={cfg}; SCUNet publishes [4,4,4,4,4,4,4]", file=sys.stderr)
    meta = {"format": "pt", "arch": "scunet", "variant": variant, "in_nc": in_nc, "dim": dim,
            "config": ",".join(str(v) for v in cfg), "head_dim": head_dim, "window_size": window}
    write_safetensors(dst, {k: state[k] for k in sorted(state)}, meta)
    return meta, len(state)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m scunet_hip.convert",
                                 description="Convert a published SCUNet .pth checkpoint into the "
                                             "safetensors file this backend and the reference crate load.")
    ap.add_argument("src")
    ap.add_argument("dst")
    ap.add_argument("--variant", default=None)
    args = ap.parse_args(argv)
    meta, n = convert(args.src, args.dst, args.variant)
    print(f"{args.dst}: {n} tensors, variant {meta['variant']}, in_nc {meta['in_nc']}, dim {meta['dim']}, "
          f"config [{meta['config']}]")
    return 0


if __name__ == "__main__":
    sys.exit(main())
