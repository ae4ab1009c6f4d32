"""The drop-in boundary on the CPU: the library builds and exports exactly what the header
declares, weight files are validated like src/weights.rs does, the plan geometry, and
the product path never reaches the oracle."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

REPO = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(REPO, "include", "scunet_hip.h")
PKG = os.path.join(REPO, "scunet-rs_amd")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(scunet_hip_\w+)\s*\(", text)))


def all_declared_symbols():
    """Every entry point of every header under include/ (the backend and the PNG codec)."""
    inc = os.path.join(REPO, "include")
    text = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    return sorted(set(re.findall(r"\b(scunet_\w+)\s*\(", text)))


def test_header_and_python_binding_agree():
    from scunet_hip import EXPORTS
    assert sorted(EXPORTS) == declared_symbols()


def test_precision_modes_match_the_header():
    """The arithmetic modes the Python mirror names are the header's #defines."""
    from scunet_hip import Hip
    text = open(os.path.join(REPO, "include", "scunet_hip.h")).read()
    defined = {m.group(1).lower(): int(m.group(2))
               for m in re.finditer(r"#define SCUNET_HIP_(FP\w+)\s+(\d+)", text)}
    assert defined == {"fp32": 0, "fp16": 1, "fp32_mfma": 2}
    assert Hip.PRECISIONS == defined


def test_library_exports_every_declared_symbol():
    from scunet_hip import LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (scunet_\w+)", out))
    assert set(declared_symbols()) < set(all_declared_symbols())
    missing = [s for s in all_declared_symbols() if s not in exported]
    assert not missing, missing
    lib = ctypes.CDLL(LIB_PATH)          # loads without a GPU: no device call at load time
    for s in all_declared_symbols():
        assert hasattr(lib, s)


def _write_bad(path, mutate):
    from scunet_hip.safetensors_io import read_safetensors, write_safetensors
    from scunet_hip import synth
    t, meta = read_safetensors(synth.weights_file(seed=0))
    t = {k: np.array(v) for k, v in t.items()}
    mutate(t, meta)
    write_safetensors(path, t, meta)


@pytest.mark.parametrize("mutate,msg", [
    (lambda t, m: m.pop("window_size"), "no `window_size` in __metadata__"),
    (lambda t, m: m.__setitem__("arch", "swin2sr"), "not `scunet`"),
    (lambda t, m: m.__setitem__("variant", "color-99"), "not one of the eight published"),
    (lambda t, m: m.__setitem__("in_nc", "1"), "implies in_nc 3"),
    (lambda t, m: m.__setitem__("config", "4,4,4"), "config has 3 entries"),
    (lambda t, m: t.__setitem__("m_body.2.conv_block.0.weight", np.zeros((256, 256, 3, 1), np.float32)),
     "m_body.2.conv_block.0.weight is [256, 256, 3, 1]"),
    (lambda t, m: t.pop("m_up2.3.trans_block.ln2.bias"), "m_up2.3.trans_block.ln2.bias"),
])
def test_create_validates_the_checkpoint_like_weights_rs(tmp_path, mutate, msg):
    """weights.rs:101-280: a malformed checkpoint fails at create with a message naming the
    field, before any device is touched (so this runs without a GPU)."""
    from scunet_hip import Hip, BackendError, LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    p = str(tmp_path / "bad.safetensors")
    _write_bad(p, mutate)
    with pytest.raises(BackendError) as e:
        Hip(p)
    assert msg in str(e.value)


def test_create_reports_a_missing_file():
    from scunet_hip import Hip, BackendError, LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    with pytest.raises(BackendError, match="No such file"):
        Hip("/nonexistent/x.safetensors")


def test_plan_geometry_and_min_size():
    # plan.rs:43-57, parity.rs:129-141.
    from scunet_hip import Plan, check_min_size, BackendError
    p = Plan(80, 64)
    assert (p.hp, p.wp) == (128, 64)
    assert Plan(256, 256).hp == 256
    assert Plan(257, 1).hp == 320
    assert Plan(1080, 1920).windows(0) == (136, 240)
    assert Plan(1080, 1920).windows(3) == (17, 30)
    check_min_size(1, 1, 8)
    with pytest.raises(BackendError):
        check_min_size(1, 1, 16)


def test_weights_generator_is_deterministic_and_loadable():
    from scunet_hip import synth
    from scunet_hip.safetensors_io import read_safetensors
    a, meta = synth.make_weights(seed=11, in_nc=1, config=(2, 2, 2, 2, 2, 2, 2))
    b, _ = synth.make_weights(seed=11, in_nc=1, config=(2, 2, 2, 2, 2, 2, 2))
    assert all(np.array_equal(a[k], b[k]) for k in a)
    assert meta["variant"].startswith("gray")
    rp = a["m_down2.1.trans_block.msa.relative_position_params"]
    assert rp.shape == (2, 15, 15) and np.abs(rp).max() <= 0.04
    t, m = read_safetensors(synth.weights_file(seed=0))
    assert m["arch"] == "scunet" and m["config"] == "4,4,4,4,4,4,4"
    assert len(t) == len(synth.tensor_specs())


def test_product_never_reaches_the_oracle():
    """Only tests/, smoke() and bench.py's CPU baseline may touch oracle/."""
    for root, _, files in os.walk(PKG):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h", "Makefile")):
                text = open(os.path.join(root, f), errors="replace").read()
                assert "oracle" not in text.lower(), os.path.join(root, f)


def _arch_of(meta):
    return {"variant": meta["variant"], "in_nc": int(meta["in_nc"]), "dim": int(meta["dim"]),
            "head_dim": int(meta["head_dim"]), "window": int(meta["window_size"]),
            "config": [int(v) for v in meta["config"].split(",")]}


@pytest.mark.parametrize("mutate", [
    lambda t, m: t.__setitem__("m_body.2.conv_block.0.weight", np.zeros((256, 256, 3, 1), np.float32)),
    lambda t, m: t.pop("m_up2.3.trans_block.ln2.bias"),
    lambda t, m: t.pop("m_down3.4.weight"),
    lambda t, m: t.__setitem__("m_up1.0.weight", np.zeros((128, 64, 2), np.float32)),
    lambda t, m: m.__setitem__("variant", "color-99"),
    lambda t, m: m.__setitem__("in_nc", "1"),
    lambda t, m: m.__setitem__("head_dim", "48"),
])
def test_create_from_tensors_fails_like_create(tmp_path, mutate):
    """scunet_hip_create_from_tensors (Cuda::new over an already-loaded Weights, cuda.rs:192)
    runs the checks of weights.rs:127-280 that scunet_hip_create runs on a file, with the
    same message (the file path replaced by "weights"), before any device is touched."""
    from scunet_hip import Hip, BackendError, LIB_PATH
    from scunet_hip.safetensors_io import read_safetensors, write_safetensors
    from scunet_hip import synth
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    t, meta = read_safetensors(synth.weights_file(seed=0))
    t = {k: np.array(v) for k, v in t.items()}
    meta = dict(meta)
    mutate(t, meta)
    p = str(tmp_path / "bad.safetensors")
    write_safetensors(p, t, meta)
    with pytest.raises(BackendError) as from_file:
        Hip(p)
    with pytest.raises(BackendError) as from_tensors:
        Hip(tensors=t, arch=_arch_of(meta))
    assert str(from_tensors.value) == str(from_file.value).replace(p, "weights")


def test_create_from_tensors_checks_its_arguments():
    from scunet_hip import Hip, BackendError, LIB_PATH
    from scunet_hip.safetensors_io import read_safetensors
    from scunet_hip import synth
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    t, meta = read_safetensors(synth.weights_file(seed=0))
    arch = _arch_of(meta)
    with pytest.raises(BackendError, match=r"config\[3\] = 0"):
        Hip(tensors=t, arch=dict(arch, config=[4, 4, 4, 0, 4, 4, 4]))
    # Extra tensors are not asked for and do not matter; a missing one is named.
    with pytest.raises(BackendError, match="weights: m_head.0.weight: no such tensor"):
        Hip(tensors={k: v for k, v in t.items() if k != "m_head.0.weight"}, arch=arch)


def _raw_safetensors(path, header):
    import json
    import struct
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        f.write(b"\0" * 64)


@pytest.mark.parametrize("shape,offsets,msg", [
    ([-1, 4], [0, 16], "not an integer in [0, 2^32]"),
    ([2.5, 4], [0, 40], "not an integer in [0, 2^32]"),
    ([2 ** 33], [0, 16], "not an integer in [0, 2^32]"),
    ([2 ** 32, 2 ** 32, 2 ** 32], [0, 16], "overflows"),
    ([4], [-16, 0], "data offsets are not non-negative integers"),
    ([4], [0, 8], "data offsets disagree with its shape"),
])
def test_header_shapes_and_offsets_are_checked(tmp_path, shape, offsets, msg):
    """A crafted header cannot make the loader size a copy from a wrapped element count."""
    from scunet_hip import Hip, BackendError, LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.skip("library not built")
    p = str(tmp_path / "crafted.safetensors")
    _raw_safetensors(p, {"x": {"dtype": "F32", "shape": shape, "data_offsets": offsets}})
    with pytest.raises(BackendError) as e:
        Hip(p)
    assert msg in str(e.value)
