"""The command-line path around the forward: the PNG codec (src/image.rs:17-69 of the
reference) and the `scunet` tool (src/main.rs).

The codec is pinned against an independent implementation, the system's libpng (called
through its simplified API with ctypes; these tests skip where it is absent): files
libpng writes (its own per-row filter choice) and files built here with each of the five
row filters forced, with and without Adam7 interlacing, decode to the pixels libpng
decodes; files the codec writes decode in libpng to the quantized values. The
quantization (image.rs:58-64: clamp to [0, 1], v * 255 + 0.5 truncated, NaN to 0) has
known answers. The GPU tests run the built `scunet` binary end to end."""
import ctypes
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

from conftest import REPO

CLI = os.path.join(REPO, "scunet-rs_amd", "lib", "scunet")

# ---------------------------------------------------------------------------
# libpng, the independent decoder/encoder (png.h's simplified API, libpng 1.6)
# ---------------------------------------------------------------------------


class _PngImage(ctypes.Structure):
    _fields_ = [("opaque", ctypes.c_void_p), ("version", ctypes.c_uint32), ("width", ctypes.c_uint32),
                ("height", ctypes.c_uint32), ("format", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("colormap_entries", ctypes.c_uint32), ("warning_or_error", ctypes.c_uint32),
                ("message", ctypes.c_char * 64)]


SPP_OF_FORMAT = {0: 1, 1: 2, 2: 3, 3: 4}   # PNG_FORMAT_GRAY, _GA, _RGB, _RGBA


@pytest.fixture(scope="module")
def libpng():
    try:
        L = ctypes.CDLL("libpng16.so.16")
    except OSError:
        pytest.skip("libpng16 is not installed")
    L.png_image_write_to_file.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p,
                                          ctypes.c_int32, ctypes.c_void_p]
    L.png_image_begin_read_from_file.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
    L.png_image_finish_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
                                        ctypes.c_void_p]
    L.png_image_free.argtypes = [ctypes.c_void_p]
    return L


def lp_write(L, path, px):
    """px: uint8 [h][w][spp] -> an 8-bit PNG written by libpng."""
    h, w, spp = px.shape
    im = _PngImage(version=1, width=w, height=h, format={1: 0, 2: 1, 3: 2, 4: 3}[spp])
    px = np.ascontiguousarray(px)
    assert L.png_image_write_to_file(ctypes.byref(im), str(path).encode(), 0, px.ctypes.data, 0, None) == 1, \
        im.message
    return path


def lp_read(L, path):
    """An 8-bit PNG decoded by libpng in the file's own format: uint8 [h][w][spp]."""
    im = _PngImage(version=1)
    assert L.png_image_begin_read_from_file(ctypes.byref(im), str(path).encode()) == 1, im.message
    spp = SPP_OF_FORMAT[im.format & 3]
    out = np.zeros((im.height, im.width, spp), np.uint8)
    ok = L.png_image_finish_read(ctypes.byref(im), None, out.ctypes.data, 0, None)
    L.png_image_free(ctypes.byref(im))
    assert ok == 1, im.message
    return out


def as_planes(px):
    """What image.rs:33-41 makes of 8-bit pixels: channels 0..c-1 (alpha dropped) / 255."""
    c = 3 if px.shape[2] >= 3 else 1
    return px[:, :, :c].transpose(2, 0, 1).astype(np.float32) / np.float32(255.0)


def make_pixels(h, w, spp, seed):
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w]
    base = (xx * 3 + yy * 2)[..., None] + np.arange(spp) * 40
    px = base + rng.integers(-20, 21, (h, w, spp))
    px[h // 3: h // 2, w // 4: w // 2] = rng.integers(0, 256, (h // 2 - h // 3, w // 2 - w // 4, spp))
    return np.clip(px, 0, 255).astype(np.uint8)


# ---------------------------------------------------------------------------
# PNG files built here, with a forced row filter (checked by libpng too)
# ---------------------------------------------------------------------------

ADAM7 = [(0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)]


def _chunk(t, body):
    return struct.pack(">I", len(body)) + t + body + struct.pack(">I", zlib.crc32(t + body) & 0xFFFFFFFF)


def _filter(rows, ftype, bpp):
    out, prev = [], np.zeros_like(rows[0], dtype=np.int32)
    for r in rows:
        r = r.astype(np.int32)
        a = np.concatenate([np.zeros(bpp, np.int32), r[:-bpp]])
        c = np.concatenate([np.zeros(bpp, np.int32), prev[:-bpp]])
        if ftype == 0:
            pred = np.zeros_like(r)
        elif ftype == 1:
            pred = a
        elif ftype == 2:
            pred = prev
        elif ftype == 3:
            pred = (a + prev) // 2
        else:
            p = a + prev - c
            pa, pb, pc = np.abs(p - a), np.abs(p - prev), np.abs(p - c)
            pred = np.where((pa <= pb) & (pa <= pc), a, np.where(pb <= pc, prev, c))
        out.append(bytes([ftype]) + ((r - pred) & 255).astype(np.uint8).tobytes())
        prev = r
    return b"".join(out)


def build_png(px, ftype, interlace=False, ctype=None, depth=8, extra=b""):
    h, w, spp = px.shape
    ctype = {1: 0, 2: 4, 3: 2, 4: 6}[spp] if ctype is None else ctype
    bpp = spp * depth // 8
    if interlace:
        raw = b"".join(_filter([px[y, x0::dx].reshape(-1) for y in range(y0, h, dy)], ftype, bpp)
                       for x0, y0, dx, dy in ADAM7 if x0 < w and y0 < h)
    else:
        raw = _filter([px[y].reshape(-1) for y in range(h)], ftype, bpp)
    ihdr = struct.pack(">IIBBBBB", w, h, depth, ctype, 0, 0, int(interlace))
    z = zlib.compress(raw, 9)
    return (b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", ihdr) + extra + _chunk(b"IDAT", z[: len(z) // 2]) +
            _chunk(b"IDAT", z[len(z) // 2:]) + _chunk(b"IEND", b""))


def filter_types(path):
    """The row filter bytes of a non-interlaced 8-bit file."""
    b = open(path, "rb").read()
    w, h, _, ctype = struct.unpack(">IIBB", b[16:26])
    spp = {0: 1, 2: 3, 4: 2, 6: 4}[ctype]
    pos, z = 8, b""
    while pos < len(b):
        n = struct.unpack(">I", b[pos:pos + 4])[0]
        if b[pos + 4:pos + 8] == b"IDAT":
            z += b[pos + 8:pos + 8 + n]
        pos += 12 + n
    raw = zlib.decompress(z)
    return {raw[r * (1 + w * spp)] for r in range(h)}


# ---------------------------------------------------------------------------
# CPU: the codec
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("spp", [1, 2, 3, 4])
def test_reads_what_libpng_writes(libpng, tmp_path, spp):
    from scunet_hip import image
    px = make_pixels(67, 129, spp, seed=spp)
    p = lp_write(libpng, tmp_path / "lp.png", px)
    assert len(filter_types(p)) >= 2          # libpng's per-row choice mixes filters
    im = image.read(p)
    assert (im.c, im.h, im.w) == ((3 if spp >= 3 else 1), 67, 129)
    assert np.array_equal(im.data, as_planes(px))


@pytest.mark.parametrize("interlace", [False, True])
@pytest.mark.parametrize("ftype", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("spp,h,w", [(3, 23, 37), (1, 9, 5), (4, 16, 19), (2, 3, 1), (3, 1, 2)])
def test_every_row_filter_and_adam7(libpng, tmp_path, ftype, interlace, spp, h, w):
    from scunet_hip import image
    px = make_pixels(h, w, spp, seed=ftype * 10 + spp)
    p = tmp_path / "f.png"
    p.write_bytes(build_png(px, ftype, interlace))
    assert np.array_equal(lp_read(libpng, p), px)      # the file says what it should
    assert np.array_equal(image.read(p).data, as_planes(px))


@pytest.mark.parametrize("c", [1, 3])
def test_libpng_reads_what_we_write(libpng, tmp_path, c):
    from scunet_hip import image
    rng = np.random.default_rng(c)
    y = rng.random((c, 41, 77), dtype=np.float32) * 1.2 - 0.1     # some values outside [0, 1]
    y[:, 5:9, 10:30] = np.linspace(0, 1, 20, dtype=np.float32)    # smooth runs: other filters win
    p = tmp_path / "out.png"
    image.write(p, y)
    got = lp_read(libpng, p)
    assert got.shape == (41, 77, c)
    want = np.floor(np.clip(y, 0, 1).astype(np.float32) * np.float32(255) + np.float32(0.5))
    assert np.array_equal(got.transpose(2, 0, 1), want.astype(np.uint8))
    assert len(filter_types(p)) >= 2
    # Reading our own file gives the quantized values back.
    assert np.array_equal(image.read(p).data, want.astype(np.float32) / np.float32(255))


def test_quantization_known_answers(tmp_path):
    """image.rs:58-64: clamp, then (u8)(v * 255 + 0.5) in float arithmetic; NaN -> 0."""
    from scunet_hip import image
    vals = [-1.0, 0.0, 0.2, 0.5, 1.0, 1.5, float("nan"), float("inf"), float("-inf"), 0.998, 0.999,
            1.0 / 255, 0.4 / 255, 0.6 / 255, 254.4 / 255, 254.6 / 255]
    want = [0, 0, 51, 128, 255, 255, 0, 255, 0, 254, 255, 1, 0, 1, 254, 255]
    p = tmp_path / "q.png"
    image.write(p, np.array(vals, np.float32).reshape(1, 1, -1))
    got = image.read(p).data.ravel() * 255
    assert np.array_equal(np.rint(got).astype(int), want)


def _write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def test_malformed_files_are_named(tmp_path):
    """Each malformed file fails with the file's name and the reason, never a wrong image."""
    from scunet_hip import image
    px = make_pixels(6, 7, 3, seed=1)
    good = build_png(px, 4)
    cases = [
        (b"GIF89a" + good[6:], "not a PNG file"),
        (good[:40], "truncated PNG"),
        (good[:-12], "no IEND"),
        (good[:45] + bytes([good[45] ^ 1]) + good[46:], "CRC mismatch in chunk IDAT"),
        (build_png(px[:, :, :1], 0, ctype=3, extra=_chunk(b"PLTE", bytes(range(6)))),
         "unsupported colour type Indexed"),
        (build_png(np.zeros((2, 2, 6), np.uint8), 0, ctype=2, depth=16), "16-bit samples"),
    ]
    for blob, msg in cases:
        p = _write(tmp_path, "bad.png", blob)
        with pytest.raises(image.ImageError, match=msg) as e:
            image.read(p)
        assert str(p) in str(e.value)
    # A row whose filter byte is not 0..4.
    ihdr = struct.pack(">IIBBBBB", 7, 1, 8, 2, 0, 0, 0)
    blob = (b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", ihdr) + _chunk(b"IDAT", zlib.compress(bytes([9]) + bytes(21))) +
            _chunk(b"IEND", b""))
    with pytest.raises(image.ImageError, match="invalid filter type 9"):
        image.read(_write(tmp_path, "f9.png", blob))
    # Too little image data for the header's geometry.
    ihdr = struct.pack(">IIBBBBB", 7, 4, 8, 2, 0, 0, 0)
    blob = (b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", ihdr) + _chunk(b"IDAT", zlib.compress(bytes(22))) +
            _chunk(b"IEND", b""))
    with pytest.raises(image.ImageError, match="image data ends early"):
        image.read(_write(tmp_path, "short.png", blob))
    # A header claiming a huge image is refused before anything is allocated for it.
    for (w, h), msg in [((1 << 15, 1 << 14), "image too large"), ((8000, 8000), "image data ends early")]:
        ihdr = struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0)
        blob = (b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", ihdr) + _chunk(b"IDAT", zlib.compress(bytes(64))) +
                _chunk(b"IEND", b""))
        with pytest.raises(image.ImageError, match=msg):
            image.read(_write(tmp_path, "huge.png", blob))
    with pytest.raises(image.ImageError, match="No such file"):
        image.read(tmp_path / "missing.png")
    with pytest.raises(image.ImageError, match="cannot write 2 channels as PNG"):
        image.write(tmp_path / "x.png", np.zeros((2, 4, 4), np.float32))


# ---------------------------------------------------------------------------
# CPU: the tool's argument handling (main.rs:50-130); nothing here reaches a device
# ---------------------------------------------------------------------------

def cli(*args, timeout=60):
    if not os.path.exists(CLI):
        pytest.skip("the scunet tool is not built")
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("args,rc,msg", [
    (["-V"], 0, "scunet 0.1.0"),
    (["--help"], 2, "USAGE:"),
    (["-m", "w", "-i", "a.png", "-o", "b.png", "--tile", "512"], 2, "`--tile` is not supported"),
    (["-m", "w", "-i", "a.png", "-o", "b.png", "--tile-pad", "8"], 2, "no tile geometry"),
    (["-m", "w", "-i", "a.png", "-o", "b.png", "--cpu"], 2, "has no cpu device"),
    (["-m", "w", "-i", "a.png", "-o", "b.png", "--device", "tpu"], 2, "unknown device `tpu`"),
    (["-i", "a.png", "-o", "b.png"], 2, "--model is required"),
    (["-m", "w", "-i", "a.png"], 2, "--input and --output are required"),
    (["-m", "w", "--frobnicate"], 2, "unknown argument `--frobnicate`"),
    (["-m"], 2, "--model needs a value"),
    (["-m", "/nonexistent.safetensors", "-i", "a.png", "-o", "b.png"], 1, "/nonexistent.safetensors"),
])
def test_cli_arguments(args, rc, msg):
    r = cli(*args)
    assert r.returncode == rc, (r.stdout, r.stderr)
    assert msg in (r.stdout + r.stderr)


# ---------------------------------------------------------------------------
# GPU: the tool end to end
# ---------------------------------------------------------------------------

@pytest.mark.gpu
def test_cli_denoises_a_png_like_backend_run(weights_path, owt, tmp_path):
    """PNG -> scunet -> PNG equals run() on the decoded image, quantized (the same library
    call), and the reference arithmetic within one 8-bit step."""
    import oracle as O
    from scunet_hip import Hip, image, synth
    x = synth.config_input(1)[:, :, :]                      # 3 x 64 x 64
    x = np.concatenate([x, x[:, :8]], axis=1)[:, :72, :]    # 72 x 64: a padded geometry
    src = tmp_path / "in.png"
    image.write(src, x)
    dst = tmp_path / "out.png"
    r = cli("-m", weights_path, "-i", src, "-o", dst, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "scunet: device hip" in r.stderr and "64x72 -> 64x72" in r.stderr
    got = image.read(dst)
    xin = image.read(src).data
    with Hip(weights_path) as be:
        y = be.run_fused(xin)
    ref = tmp_path / "ref.png"
    image.write(ref, y)
    assert np.array_equal(got.data, image.read(ref).data)
    want = O.run(owt, xin)
    q = np.floor(np.clip(want, 0, 1) * np.float32(255) + np.float32(0.5)) / 255
    assert np.abs(got.data - q).max() <= 1.0 / 255 + 1e-6


@pytest.mark.gpu
def test_cli_rgba_gray_fp16_and_channel_refusal(weights_path, weights_path_gray, tmp_path, libpng):
    from scunet_hip import image
    px = make_pixels(64, 80, 4, seed=9)
    rgba = lp_write(libpng, tmp_path / "rgba.png", px)
    rgb = lp_write(libpng, tmp_path / "rgb.png", np.ascontiguousarray(px[:, :, :3]))
    a, b = tmp_path / "a.png", tmp_path / "b.png"
    assert cli("-q", "-m", weights_path, "-i", rgba, "-o", a, timeout=120).returncode == 0
    assert cli("-q", "-m", weights_path, "-i", rgb, "-o", b, timeout=120).returncode == 0
    assert np.array_equal(image.read(a).data, image.read(b).data)        # alpha dropped
    f16 = tmp_path / "f16.png"
    r = cli("-m", weights_path, "-i", rgb, "-o", f16, "--fp16", timeout=120)
    assert r.returncode == 0 and "fp16 operands" in r.stderr
    # fp16 operands: within 4e-3 of fp32 before quantization, so at most 2 steps after.
    assert np.abs(image.read(f16).data - image.read(b).data).max() <= 2.0 / 255 + 1e-6
    r = cli("-m", weights_path_gray, "-i", rgb, "-o", a, timeout=120)
    assert r.returncode == 2 and "3 channels, but this checkpoint takes 1" in r.stderr
    gray = lp_write(libpng, tmp_path / "g.png", np.ascontiguousarray(px[:, :, :1]))
    r = cli("-q", "-m", weights_path_gray, "-i", gray, "-o", a, timeout=120)
    assert r.returncode == 0, r.stderr
    assert image.read(a).c == 1
