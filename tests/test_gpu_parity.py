"""The HIP backend against the oracle (the C++ restatement of the reference's src/cpu.rs),
op by op, block by block and end to end, through the C ABI. Modeled on the reference's
tests/cuda_ops.rs: every primitive is compared on the same synthetic input against the
cpu.rs function it corresponds to, so a failure names the kernel.

Tolerances: the north star's per-stage bar is max |diff| <= 1e-4 against the reference's
fp32 path; the per-op checks use the reference's own structural bound (worst |diff|
within tol x the data's magnitude, tests/cuda_ops.rs:49-73), tightened where the device
computes the same sums in a different order only.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import close, max_abs

pytestmark = pytest.mark.gpu

STAGE_TOL = 1e-4        # north star: per stage, against the reference fp32 path


@pytest.fixture(scope="module")
def be(weights_path):
    from scunet_hip import Hip
    h = Hip(weights_path)
    yield h
    h.close()


@pytest.fixture(scope="module")
def be_affine(weights_path_affine):
    from scunet_hip import Hip
    h = Hip(weights_path_affine)
    yield h
    h.close()


@pytest.fixture(scope="module")
def owt_affine(weights_path_affine):
    return O.Weights.load(weights_path_affine)


def seq(n, a):
    from scunet_hip.synth import seq as s
    return s(n, a)


def to_tokens(plane, c, n):
    return np.ascontiguousarray(plane.reshape(c, n).T)


# ---------------------------------------------------------------------------
# Construction and the trait surface
# ---------------------------------------------------------------------------

def test_backend_identity(be):
    assert be.name() == "hip"
    assert (be.in_nc, be.dim, be.head_dim, be.window) == (3, 64, 32, 8)
    assert be.config == [4] * 7
    w, _ = be.footprint()
    assert w >= 4 * 18_000_000          # the whole checkpoint is resident after create


def test_create_from_tensors_equals_create_from_file(be, weights_path):
    """scunet_hip_create_from_tensors (Cuda::new over the caller's loaded Weights,
    cuda.rs:192-241): the same network, bit for bit, as the handle that read the file, and
    the caller's buffers are not needed after the call."""
    from scunet_hip import Hip, run
    from scunet_hip.safetensors_io import read_safetensors
    from scunet_hip import synth
    t, meta = read_safetensors(weights_path)
    t = {k: np.array(v) for k, v in t.items()}
    arch = {"variant": meta["variant"], "in_nc": 3, "dim": 64, "head_dim": 32, "window": 8,
            "config": [4] * 7}
    x = synth.config_input(1)
    with Hip(tensors=t, arch=arch) as h2:
        for v in t.values():
            v[...] = np.nan            # the library copied what it needed during create
        assert (h2.in_nc, h2.dim, h2.head_dim, h2.window, h2.config) == (3, 64, 32, 8, [4] * 7)
        assert h2.variant == meta["variant"]
        assert be.footprint()[0] == h2.footprint()[0]
        assert np.array_equal(run(be, x), run(h2, x))


def test_forward_rejects_wrong_shapes(be):
    from scunet_hip import BackendError, Plan
    with pytest.raises(BackendError):
        be.forward(np.zeros((3, 64, 64), np.float32), Plan(64, 128))
    with pytest.raises(BackendError, match="channels"):
        be.run_fused(np.zeros((1, 64, 64), np.float32))


# ---------------------------------------------------------------------------
# Ops against their cpu.rs twins (cuda_ops.rs:254-317)
# ---------------------------------------------------------------------------

def test_conv1x1_matches_cpu(be, owt):
    h, w = 16, 24
    for name, c in (("m_down1.0.conv1_1", 64), ("m_body.2.conv1_2", 512)):
        x = seq(c * h * w, 0.31).reshape(c, h, w)
        got = be.op_probe("conv1x1", name, x, c, c, h, w)
        want = O.conv1x1(x, owt.t[name + ".weight"].reshape(c, c), owt.t[name + ".bias"])
        close(f"conv1x1 {name}", want, got, 1e-5)


def test_conv3x3_matches_cpu(be, owt):
    h, w = 16, 24
    for name, c in (("m_down1.0.conv_block.0", 32), ("m_down2.1.conv_block.2", 64),
                    ("m_body.0.conv_block.0", 256)):
        x = seq(c * h * w, 0.37).reshape(c, h, w)
        got = be.op_probe("conv3x3", name, x, c, c, h, w)
        want = O.conv3x3(x, owt.t[name + ".weight"])
        close(f"conv3x3 {name}", want, got, 1e-5)
    # Odd geometry: partial 16x16 tiles on both axes.
    x = seq(32 * 40 * 24, 0.41).reshape(32, 40, 24)
    got = be.op_probe("conv3x3", "m_up1.1.conv_block.0", x, 32, 32, 40, 24)
    close("conv3x3 40x24", O.conv3x3(x, owt.t["m_up1.1.conv_block.0.weight"]), got, 1e-5)


def test_head_and_tail_match_cpu(be, owt):
    h, w = 24, 40
    x = seq(3 * h * w, 0.5).reshape(3, h, w)
    got = be.op_probe("conv3x3", "m_head.0", x, 3, 64, h, w)
    want = O.conv3x3(x, owt.t["m_head.0.weight"])
    close("m_head", want, got, 1e-6)
    y = seq(64 * h * w, 0.45).reshape(64, h, w)
    got = be.op_probe("conv3x3", "m_tail.0", y, 64, 3, h, w)
    close("m_tail", O.conv3x3(y, owt.t["m_tail.0.weight"]), got, 1e-5)


def test_stride2_and_transposed_match_cpu(be, owt):
    h, w = 16, 24
    for name, ci in (("m_down1.4", 64), ("m_down3.4", 256)):
        x = seq(ci * h * w, 0.33).reshape(ci, h, w)
        got = be.op_probe("conv2x2s2", name, x, ci, 2 * ci, h, w)
        close(f"conv2x2s2 {name}", O.conv2x2s2(x, owt.t[name + ".weight"]), got, 1e-5)
    for name, ci in (("m_up3.0", 512), ("m_up1.0", 128)):
        x = seq(ci * 8 * 16, 0.35).reshape(ci, 8, 16)
        got = be.op_probe("conv_t2x2", name, x, ci, ci // 2, 8, 16)
        close(f"conv_t2x2 {name}", O.conv_t2x2(x, owt.t[name + ".weight"]), got, 1e-5)


def test_linear_against_row_major_matmul(be, owt):
    # cuda_ops.rs:279-297: rows not a multiple of any tile.
    for rows, name in ((5, "m_body.0.trans_block.msa.linear"), (333, "m_down2.0.trans_block.mlp.0"),
                       (130, "m_up3.2.trans_block.mlp.2")):
        wt, b = owt.t[name + ".weight"], owt.t[name + ".bias"]
        co, ci = wt.shape
        x = seq(rows * ci, 0.29).reshape(rows, ci)
        got = be.linear_probe(name, x, rows, ci, co)
        want = x.astype(np.float64) @ wt.T.astype(np.float64) + b
        close(f"linear {name}", want, got, 1e-5)


def test_layer_norm_closed_form(be_affine, owt_affine):
    for rows, name in ((7, "m_down1.0.trans_block.ln1"), (300, "m_body.1.trans_block.ln2"),
                       (129, "m_down2.3.trans_block.ln1")):
        g, b = owt_affine.t[name + ".weight"], owt_affine.t[name + ".bias"]
        c = g.size
        x = (seq(rows * c, 0.41) * 3 + 0.5).reshape(rows, c)
        got = be_affine.layer_norm_probe(name, x, rows, c)
        close(f"layer_norm {name}", O.layer_norm(x, g, b), got, 1e-5)


# ---------------------------------------------------------------------------
# The window index map (cuda_ops.rs:322-359)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("h,w,c,shift", [(8, 8, 32, 0), (16, 16, 32, 4), (16, 16, 8, 0), (32, 24, 4, 4),
                                         (32, 24, 4, 0), (24, 32, 4, 4)])
def test_window_index_map(be, h, w, c, shift):
    x = seq(c * h * w, 0.61).reshape(c, h, w)
    rt = be.window_round_trip(h, w, c, shift, x)
    assert np.array_equal(rt.ravel(), x.ravel())
    nww, nn = w // 8, 64
    want = np.zeros(((h // 8) * nww * nn, c), np.float32)
    for wi in range((h // 8) * nww):
        wh, ww = divmod(wi, nww)
        for t in range(nn):
            i, j = divmod(t, 8)
            y, xx = (wh * 8 + i + shift) % h, (ww * 8 + j + shift) % w
            want[wi * nn + t] = x[:, y, xx]
    assert np.array_equal(be.gather_probe(h, w, c, shift, x).reshape(want.shape), want)


# ---------------------------------------------------------------------------
# The attention kernel (cuda_ops.rs:365-450 known answers + a float64 evaluation)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("h,w", [(8, 8), (16, 8), (16, 16)])
def test_attention_uniform_case(be, h, w):
    c, heads, hd = 32, 1, 32
    nt = (h // 8) * (w // 8) * 64
    qkv = np.zeros((nt, 3 * c), np.float32)
    qkv[:, :c] = 1.0
    t = np.arange(nt)
    qkv[:, 2 * c:] = 2.0
    qkv[:, 2 * c] = (t % 17).astype(np.float32)
    got = be.attention_kernel_probe(h, w, c, heads, hd, 0, qkv, np.zeros((1, 15, 15), np.float32))
    want = np.zeros((nt, c), np.float32)
    for wi in range(nt // 64):
        blk = qkv[wi * 64:(wi + 1) * 64, 2 * c:]
        want[wi * 64:(wi + 1) * 64] = blk.astype(np.float64).mean(0)
    close(f"uniform attention {h}x{w}", want, got, 1e-5)


def test_attention_known_softmax(be):
    c, hd = 32, 32
    qkv = np.zeros((64, 3 * c), np.float32)
    t = np.arange(64)
    qkv[:, 0] = 1.0
    qkv[t, c + (t % hd)] = 1.0
    qkv[:, 2 * c] = 3.0
    qkv[:, 2 * c + 1] = 1.0
    got = be.attention_kernel_probe(8, 8, c, 1, hd, 0, qkv, np.zeros((1, 15, 15), np.float32)).reshape(64, c)
    scale = 1.0 / math.sqrt(hd)
    e = np.where(t % hd == 0, math.exp(scale), 1.0)
    want = np.zeros((64, c))
    want[:, 0] = 3.0 * e.sum() / e.sum()
    want[:, 1] = 1.0 * e.sum() / e.sum()
    close("known softmax", want, got, 1e-5)


def _attn_core_f64(qkv, rp, h, w, c, heads, shift):
    """Upstream WMSA core (network_scunet.py:84-97) on window-major qkv, float64."""
    ws = 8
    nwh, nww = h // ws, w // ws
    cord = np.array([[i, j] for i in range(ws) for j in range(ws)])
    rel = cord[:, None, :] - cord[None, :, :] + ws - 1
    q = qkv.reshape(nwh * nww, 64, 3 * c).astype(np.float64)
    out = np.zeros((nwh * nww, 64, c))
    mask = np.zeros((nwh, nww, 8, 8, 8, 8), bool)
    if shift:
        s = 4
        mask[-1, :, :s, :, s:, :] = True
        mask[-1, :, s:, :, :s, :] = True
        mask[:, -1, :, :s, :, s:] = True
        mask[:, -1, :, s:, :, :s] = True
    mask = mask.reshape(nwh * nww, 64, 64)
    for hh in range(heads):
        qq = q[..., hh * 32:(hh + 1) * 32]
        kk = q[..., c + hh * 32:c + (hh + 1) * 32]
        vv = q[..., 2 * c + hh * 32:2 * c + (hh + 1) * 32]
        sim = qq @ kk.transpose(0, 2, 1) * 32 ** -0.5 + rp[hh][rel[..., 0], rel[..., 1]]
        sim = np.where(mask, -np.inf, sim)
        e = np.exp(sim - sim.max(-1, keepdims=True))
        out[..., hh * 32:(hh + 1) * 32] = (e / e.sum(-1, keepdims=True)) @ vv
    return out.reshape(-1, c)


@pytest.mark.parametrize("h,w,c,shift", [(8, 8, 32, 0), (16, 24, 32, 4), (24, 16, 64, 4), (16, 16, 128, 0),
                                         (16, 16, 256, 4), (32, 40, 64, 4)])
def test_attention_kernel_against_float64(be, h, w, c, shift):
    heads = c // 32
    rng = np.random.default_rng(h * 1000 + w + c + shift)
    nt = (h // 8) * (w // 8) * 64
    qkv = rng.standard_normal((nt, 3 * c)).astype(np.float32)
    rp = (rng.standard_normal((heads, 15, 15)) * 0.5).astype(np.float32)
    got = be.attention_kernel_probe(h, w, c, heads, 32, shift, qkv, rp)
    want = _attn_core_f64(qkv, rp, h, w, c, heads, shift)
    assert max_abs(want, got) < 2e-5, (h, w, c, shift)


@pytest.mark.parametrize("prefix,h,w,shift", [("m_down1.0", 8, 8, 0), ("m_down1.0", 16, 16, 0),
                                              ("m_down1.0", 16, 16, 4), ("m_down2.0", 16, 16, 4),
                                              ("m_body.0", 16, 16, 0), ("m_body.0", 16, 16, 4)])
def test_attention_probe_matches_cpu_attention(be, owt, prefix, h, w, shift):
    # cuda_ops.rs:528-585: gather + LN1 + qkv + attention + proj against cpu::attention.
    tp = prefix + ".trans_block"
    c = owt.t[tp + ".ln1.weight"].size
    n = h * w
    plane = seq(c * n, 0.43).reshape(c, h, w)
    tok = be.attention_probe(prefix, h, w, c, shift, plane).reshape(-1, c)
    ln = O.layer_norm(to_tokens(plane, c, n), owt.t[tp + ".ln1.weight"], owt.t[tp + ".ln1.bias"])
    g = lambda s: owt.t[f"{tp}.msa.{s}"]
    want = O.attention(ln, h, w, c, 8, shift, g("embedding_layer.weight"), g("embedding_layer.bias"),
                       g("linear.weight"), g("linear.bias"), g("relative_position_params"))
    got = np.zeros((n, c), np.float32)
    hits = np.zeros(n, int)
    nww = w // 8
    for wi in range((h // 8) * nww):
        wh, ww = divmod(wi, nww)
        for t in range(64):
            i, j = divmod(t, 8)
            y, xx = (wh * 8 + i + shift) % h, (ww * 8 + j + shift) % w
            got[y * w + xx] = tok[wi * 64 + t]
            hits[y * w + xx] += 1
    assert (hits == 1).all()
    close(f"attention probe {prefix} {h}x{w} shift{shift}", want, got, 2e-5)


# ---------------------------------------------------------------------------
# Blocks (cuda_ops.rs:129-251)
# ---------------------------------------------------------------------------

BLOCK_CASES = [("m_body.0", 32, 16, 0), ("m_body.0", 16, 32, 0), ("m_body.0", 32, 32, 0), ("m_body.0", 64, 16, 0),
               ("m_body.0", 16, 16, 0), ("m_body.0", 32, 16, 4), ("m_body.0", 16, 32, 4), ("m_body.0", 32, 32, 4),
               ("m_body.0", 16, 16, 4), ("m_body.0", 8, 8, 4), ("m_down1.0", 16, 16, 0), ("m_down1.0", 16, 16, 4),
               ("m_down2.0", 16, 16, 0), ("m_up1.2", 24, 40, 4), ("m_up2.3", 40, 24, 0)]


@pytest.mark.parametrize("prefix,h,w,shift", BLOCK_CASES)
def test_block_matches_cpu(be, owt, prefix, h, w, shift):
    c = sum(owt.block_dims(prefix))
    x = seq(c * h * w, 0.53).reshape(c, h, w)
    got = be.block_dump(prefix, h, w, shift, x)
    want = O.conv_trans_block(owt, prefix, x, shift)
    assert max_abs(want, got) <= STAGE_TOL
    close(f"{prefix} {h}x{w} shift{shift}", want, got, 3e-5)


@pytest.mark.parametrize("prefix,h,w,shift", [("m_body.0", 576, 64, 0), ("m_body.0", 576, 64, 4),
                                              ("m_down1.0", 512, 72, 0), ("m_down1.0", 512, 72, 4)])
def test_block_past_the_token_budget(be, owt, prefix, h, w, shift):
    # cuda_ops.rs:175-195: planes larger than the reference's 512-window chunk.
    c = sum(owt.block_dims(prefix))
    x = seq(c * h * w, 0.71).reshape(c, h, w)
    got = be.block_dump(prefix, h, w, shift, x)
    want = O.conv_trans_block(owt, prefix, x, shift)
    assert max_abs(want, got) <= STAGE_TOL
    close(f"{prefix} {h}x{w} shift{shift}", want, got, 3e-5)


def test_block_with_random_layernorm_affine(be_affine, owt_affine):
    for prefix, shift in (("m_down1.1", 4), ("m_body.2", 0)):
        c = sum(owt_affine.block_dims(prefix))
        x = seq(c * 16 * 24, 0.57).reshape(c, 16, 24)
        got = be_affine.block_dump(prefix, 16, 24, shift, x)
        want = O.conv_trans_block(owt_affine, prefix, x, shift)
        close(f"affine LN {prefix}", want, got, 3e-5)


def test_block_repeats_are_bit_identical(be):
    # cuda_ops.rs:217-251: the device against itself, a race detector.
    for prefix, h, w, shift in (("m_body.0", 576, 64, 0), ("m_body.0", 576, 64, 4)):
        c = 512
        x = seq(c * h * w, 0.71).reshape(c, h, w)
        first = be.block_dump(prefix, h, w, shift, x)
        for r in range(1, 12):
            got = be.block_dump(prefix, h, w, shift, x)
            assert np.array_equal(first, got), f"{prefix} shift{shift}: run {r} differs from run 0"


# ---------------------------------------------------------------------------
# End to end (cuda_ops.rs:98-124, 616-635; parity.rs)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("h,w", [(64, 64), (128, 64), (80, 64), (96, 64), (72, 40), (64, 80), (100, 100)])
def test_forward_matches_cpu_backend(be, owt, h, w):
    from scunet_hip import run
    x = seq(3 * h * w, 0.7).reshape(3, h, w)
    want = O.run(owt, x)
    got = run(be, x)
    assert max_abs(want, got) <= STAGE_TOL, (h, w)
    fused = be.run_fused(x)                 # pad + crop on the device
    assert max_abs(want, fused) <= STAGE_TOL, (h, w)
    assert np.array_equal(got, fused)


def test_every_stage_within_1e4_at_64x64(be, owt, golden):
    x = golden["fwd64_in"]
    _, want = O.forward_dump(owt, x)
    got = {}
    y = be.forward_dump(x, lambda n, v: got.__setitem__(n, v))
    assert list(got) == list(want)
    for name in want:
        d = max_abs(want[name], got[name])
        assert d <= STAGE_TOL, f"{name}: {d:.3e}"
    assert max_abs(golden["fwd64_out"], y) <= STAGE_TOL


def test_forward_against_reference_py_golden(be, golden):
    from scunet_hip import run
    for key in ("fwd64", "fwd80x72"):
        got = run(be, golden[f"{key}_in"])
        assert max_abs(golden[f"{key}_out"], got) <= STAGE_TOL, key


def test_forward_past_the_token_budget_256(be, owt):
    from scunet_hip import run
    x = seq(3 * 256 * 256, 0.31).reshape(3, 256, 256)
    want = O.run(owt, x)
    got = run(be, x)
    assert max_abs(want, got) <= STAGE_TOL


def test_forward_device_entry_and_release(be, owt):
    x = seq(3 * 128 * 192, 0.37).reshape(3, 128, 192)
    want = O.run(owt, x)
    xp = be.malloc(x.nbytes)
    yp = be.malloc(x.nbytes)
    try:
        be.h2d(xp, x)
        be.forward_device(xp, 3, 128, 192, yp)
        got = be.d2h(np.empty_like(x), yp)
    finally:
        be.free(xp)
        be.free(yp)
    assert max_abs(want, got) <= STAGE_TOL
    be.release_scratch()
    assert be.footprint()[1] == 0
