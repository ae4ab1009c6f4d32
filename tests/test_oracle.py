"""The CPU oracle pinned against the reference's golden vectors, closed forms and
library routines. A plausible mistake in the restatement (a dropped term, a wrong
index or sign, a transposed operand, the wrong padding) fails at least one of these.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import close, max_abs


# ---------------------------------------------------------------------------
# End-to-end composition: golden vectors from tools/reference.py
# ---------------------------------------------------------------------------

def test_golden_was_made_with_this_checkpoint(golden, owt):
    from make_golden import weights_check
    assert np.allclose(weights_check(owt.t), golden["weights_check"], rtol=0, atol=1e-9)


def test_forward_matches_reference_py(golden, owt):
    # reference.py pads, walks and crops; O.run does the same as backend.rs:63-105.
    for key in ("fwd64", "fwd80x72"):
        got = O.run(owt, golden[f"{key}_in"])
        assert max_abs(golden[f"{key}_out"], got) <= 1e-5, key


def test_stages_match_reference_py(golden, owt):
    from make_golden import STAGES, sample_idx
    _, st = O.forward_dump(owt, golden["fwd64_in"])
    assert list(st) == STAGES          # the 16 hook names, in cpu.rs's order
    for i, name in enumerate(STAGES):
        v = st[name]
        idx = sample_idx(v.size, 2048, 1000 + i)
        assert max_abs(golden[f"stage64_{name}_val"], v[idx]) <= 1e-5, name
        s = golden[f"stage64_{name}_stats"]
        assert abs(np.abs(v).max() - s[0]) <= 1e-5, name


def test_blocks_match_reference_py(golden, owt):
    from make_golden import BLOCK_CASES
    from scunet_hip import synth
    for k, (prefix, h, w, shifted) in enumerate(BLOCK_CASES):
        c = owt.t[f"{prefix}.conv1_1.weight"].shape[0]
        x = synth.seq(c * h * w, 0.53 + 0.01 * k).reshape(c, h, w)
        assert abs(x.astype(np.float64).sum() - golden[f"blk_{k}_insum"][0]) < 1e-6
        got = O.conv_trans_block(owt, prefix, x, 4 if shifted else 0)
        assert max_abs(golden[f"blk_{k}_out"], got) <= 5e-6, prefix


def test_window_attention_matches_reference_py(golden, owt):
    from make_golden import WMSA_CASES
    from scunet_hip import synth
    for k, (prefix, h, w, shifted) in enumerate(WMSA_CASES):
        tp = prefix + ".trans_block"
        t = owt.t[f"{tp}.msa.linear.weight"].shape[0]
        x = synth.seq(h * w * t, 0.43 + 0.01 * k).reshape(h * w, t)
        ln = O.layer_norm(x, owt.t[tp + ".ln1.weight"], owt.t[tp + ".ln1.bias"])
        g = lambda s: owt.t[f"{tp}.msa.{s}"]
        got = O.attention(ln, h, w, t, 8, 4 if shifted else 0, g("embedding_layer.weight"),
                          g("embedding_layer.bias"), g("linear.weight"), g("linear.bias"),
                          g("relative_position_params"))
        assert max_abs(golden[f"wmsa_{k}_out"].reshape(h * w, t), got) <= 1e-6, prefix


# ---------------------------------------------------------------------------
# Ops against their definitions (brute force) and against torch (a library)
# ---------------------------------------------------------------------------

def _conv_direct(x, wt, pad, stride):
    c_in, h, w = x.shape
    c_out, _, kh, kw = wt.shape
    xp = np.pad(x.astype(np.float64), ((0, 0), (pad, pad), (pad, pad)))
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (w + 2 * pad - kw) // stride + 1
    out = np.zeros((c_out, oh, ow))
    for co in range(c_out):
        for y in range(oh):
            for xx in range(ow):
                patch = xp[:, y * stride:y * stride + kh, xx * stride:xx * stride + kw]
                out[co, y, xx] = (patch * wt[co]).sum()
    return out


def test_conv3x3_zero_padding_bruteforce():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 5, 7)).astype(np.float32)
    wt = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    got = O.conv3x3(x, wt)
    assert max_abs(_conv_direct(x, wt, 1, 1), got) < 1e-5
    # Replicate padding here would be the network's other padding - and wrong.
    xr = np.pad(x, ((0, 0), (1, 1), (1, 1)), mode="edge")
    assert max_abs(_conv_direct(xr, wt, 0, 1), got) > 1e-2


def test_conv3x3_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    x = rng.standard_normal((32, 12, 20)).astype(np.float32)
    wt = (rng.standard_normal((16, 32, 3, 3)) * 0.1).astype(np.float32)
    want = torch.nn.functional.conv2d(torch.from_numpy(x)[None].double(),
                                      torch.from_numpy(wt).double(), padding=1)[0].numpy()
    assert max_abs(want, O.conv3x3(x, wt)) < 2e-5


def test_conv2x2s2_bruteforce_and_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    x = rng.standard_normal((8, 6, 10)).astype(np.float32)
    wt = rng.standard_normal((16, 8, 2, 2)).astype(np.float32)
    got = O.conv2x2s2(x, wt)
    assert max_abs(_conv_direct(x, wt, 0, 2), got) < 1e-5
    want = torch.nn.functional.conv2d(torch.from_numpy(x)[None].double(),
                                      torch.from_numpy(wt).double(), stride=2)[0].numpy()
    assert max_abs(want, got) < 1e-5


def test_conv1x1_is_a_channel_matmul():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((12, 9, 11)).astype(np.float32)
    wt = rng.standard_normal((10, 12)).astype(np.float32)
    b = rng.standard_normal(10).astype(np.float32)
    got = O.conv1x1(x, wt, b)
    want = np.einsum("oi,ihw->ohw", wt.astype(np.float64), x) + b[:, None, None]
    assert max_abs(want, got) < 1e-5


def test_conv_t2x2_no_tap_flip_bruteforce_and_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 4, 5)).astype(np.float32)
    wt = rng.standard_normal((6, 3, 2, 2)).astype(np.float32)     # [c_in][c_out][2][2]
    got = O.conv_t2x2(x, wt)
    want = np.zeros((3, 8, 10))
    for ci in range(6):
        for co in range(3):
            for i in range(4):
                for j in range(5):
                    for dy in range(2):
                        for dx in range(2):
                            want[co, 2 * i + dy, 2 * j + dx] += wt[ci, co, dy, dx] * x[ci, i, j]
    assert max_abs(want, got) < 1e-5
    tw = torch.nn.functional.conv_transpose2d(torch.from_numpy(x)[None].double(),
                                              torch.from_numpy(wt).double(), stride=2)[0].numpy()
    assert max_abs(tw, got) < 1e-5
    flipped = np.zeros_like(want)
    for dy in range(2):
        for dx in range(2):
            flipped[:, dy::2, dx::2] = want[:, 1 - dy::2, 1 - dx::2]
    assert max_abs(flipped, got) > 1e-2


def test_layer_norm_closed_form():
    rng = np.random.default_rng(10)
    for c in (32, 64, 256):
        x = (rng.standard_normal((7, c)) * 3 + 1).astype(np.float32)
        g = rng.standard_normal(c).astype(np.float32)
        b = rng.standard_normal(c).astype(np.float32)
        xd = x.astype(np.float64)
        mu = xd.mean(-1, keepdims=True)
        var = ((xd - mu) ** 2).mean(-1, keepdims=True)
        want = (xd - mu) / np.sqrt(var + 1e-5) * g + b
        close(f"layer_norm c={c}", want, O.layer_norm(x, g, b), 1e-5)


def test_erf_and_gelu_against_math_erf():
    xs = np.linspace(-6, 6, 2401)
    worst = max(abs(O.erf(v) - math.erf(v)) for v in xs)
    assert worst < 1.5e-7                       # the A&S 7.1.26 bound (cpu.rs:319)
    assert O.erf(0.3) == -O.erf(-0.3)
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert max_abs(want, O.gelu(x)) < 1e-6


def test_rel_pos_table_matches_upstream_construction():
    # network_scunet.py:104-108: cord = [[i, j] ...]; relation = cord[:,None] - cord[None] + ws-1;
    # table[p][q] = params[relation[p,q,0], relation[p,q,1]].
    ws = 8
    rng = np.random.default_rng(11)
    params = rng.standard_normal((15, 15)).astype(np.float32)
    cord = np.array([[i, j] for i in range(ws) for j in range(ws)])
    rel = cord[:, None, :] - cord[None, :, :] + ws - 1
    want = params[rel[..., 0], rel[..., 1]]
    assert np.array_equal(O.rel_pos_table(params, ws), want)
    # The flattened-cord reading (the trap cpu.rs:529-531 describes) is different.
    flat = np.arange(ws * ws)
    wrong = params.ravel()[(flat[:, None] - flat[None, :] + ws * ws - 1) % params.size]
    assert not np.array_equal(want, wrong)


def _upstream_mask(nwh, nww, p=8, shift=4):
    # network_scunet.py:49-66, generate_mask for type 'SW'.
    s = p - shift
    m = np.zeros((nwh, nww, p, p, p, p), bool)
    m[-1, :, :s, :, s:, :] = True
    m[-1, :, s:, :, :s, :] = True
    m[:, -1, :, :s, :, s:] = True
    m[:, -1, :, s:, :, :s] = True
    return m.reshape(nwh * nww, p * p, p * p)


def test_mask_matches_upstream_slice_rules():
    nwh, nww = 3, 3
    want = _upstream_mask(nwh, nww)
    for wi in range(nwh * nww):
        wh, ww = divmod(wi, nww)
        got = np.array([[O.mask_hit(p, t, wh, ww, nwh, nww, 8) for t in range(64)]
                        for p in range(64)])
        assert np.array_equal(got, want[wi]), wi
    # No row of the mask is ever fully masked (the finite sentinel never meets an empty row).
    assert not want.all(axis=-1).any()


def test_attention_bruteforce_float64():
    """cpu.rs:602-758 against a direct float64 evaluation of upstream's WMSA.forward."""
    rng = np.random.default_rng(12)
    h, w, c, heads, ws = 16, 24, 64, 2, 8
    x = rng.standard_normal((h, w, c)).astype(np.float32)
    emb_w = (rng.standard_normal((3 * c, c)) * 0.2).astype(np.float32)
    emb_b = (rng.standard_normal(3 * c) * 0.1).astype(np.float32)
    lin_w = (rng.standard_normal((c, c)) * 0.2).astype(np.float32)
    lin_b = (rng.standard_normal(c) * 0.1).astype(np.float32)
    rp = (rng.standard_normal((heads, 15, 15)) * 0.5).astype(np.float32)
    cord = np.array([[i, j] for i in range(ws) for j in range(ws)])
    rel = cord[:, None, :] - cord[None, :, :] + ws - 1
    for shift in (0, 4):
        xr = np.roll(x.astype(np.float64), (-shift, -shift), axis=(0, 1))
        nwh, nww = h // ws, w // ws
        xt = xr.reshape(nwh, ws, nww, ws, c).transpose(0, 2, 1, 3, 4).reshape(nwh * nww, 64, c)
        qkv = xt @ emb_w.T.astype(np.float64) + emb_b
        out = np.zeros((nwh * nww, 64, c))
        mask = _upstream_mask(nwh, nww) if shift else np.zeros((nwh * nww, 64, 64), bool)
        for hd in range(heads):
            q = qkv[..., hd * 32:(hd + 1) * 32]
            k = qkv[..., c + hd * 32:c + (hd + 1) * 32]
            v = qkv[..., 2 * c + hd * 32:2 * c + (hd + 1) * 32]
            sim = q @ k.transpose(0, 2, 1) * 32 ** -0.5 + rp[hd][rel[..., 0], rel[..., 1]]
            sim = np.where(mask, -np.inf, sim)
            e = np.exp(sim - sim.max(-1, keepdims=True))
            out[..., hd * 32:(hd + 1) * 32] = (e / e.sum(-1, keepdims=True)) @ v
        out = out @ lin_w.T.astype(np.float64) + lin_b
        out = out.reshape(nwh, nww, ws, ws, c).transpose(0, 2, 1, 3, 4).reshape(h, w, c)
        out = np.roll(out, (shift, shift), axis=(0, 1))
        got = O.attention(x.reshape(h * w, c), h, w, c, ws, shift, emb_w, emb_b, lin_w, lin_b, rp)
        assert max_abs(out.reshape(h * w, c), got) < 2e-5, shift


def test_pad_crop_and_plan_geometry():
    # plan.rs:43-47 and tests/parity.rs:129-141.
    assert O.plan(80, 64) == (128, 64)
    assert O.plan(256, 256) == (256, 256)
    assert O.plan(257, 1) == (320, 64)
    assert O.plan(1080, 1920) == (1088, 1920)
    rng = np.random.default_rng(13)
    x = rng.random((3, 5, 7)).astype(np.float32)
    p = O.pad_replicate(x, 8, 9)
    assert np.array_equal(p, np.pad(x, ((0, 0), (0, 3), (0, 2)), mode="edge"))
    assert np.array_equal(O.crop(p, 5, 7), x)


def test_missing_weight_raises_instead_of_aborting(owt):
    # The oracle shares its process with the GPU test session: a missing tensor must surface
    # as a Python exception naming it, not end the process.
    t = {k: v for k, v in owt.t.items() if k != "m_down1.0.conv1_2.bias"}
    wt = O.Weights(t, owt.meta)
    x = np.zeros((64, 64, 64), np.float32)
    with pytest.raises(RuntimeError, match="m_down1.0.conv1_2.bias"):
        O.conv_trans_block(wt, "m_down1.0", x, 0)
    with pytest.raises(RuntimeError, match="m_down1.0.conv1_2.bias"):
        O.forward(wt, np.zeros((3, 64, 64), np.float32))
