"""The reference's golden-fixture container ("SCUF"), read and written.

Layout (src/fixture.rs:1-117 reads it, tools/make_fixture.py:8-16 writes it), all
little-endian:

    magic   b"SCUF"                         4 bytes
    version u32                             1
    h, w, c, win                            u32 each
    vlen    u32                             length of the variant string
    variant utf-8                           vlen bytes
    input   f32[c*h*w]                      NCHW, the values the network sees
    output  f32[c*h*w]                      what the reference produced (uncropped)

`Fixture.load` rejects the same malformed files as fixture.rs:37-80, with the same
messages (a wrong magic, another version, a variant string longer than the file, a
payload of the wrong size). `compare` and `locate` are fixture.rs:85-117: the worst
absolute difference, its flat index and the mean, and an index as (y, x, channel).
"""
import struct

import numpy as np

MAGIC = b"SCUF"

__all__ = ["MAGIC", "Fixture", "save"]


class Fixture:
    def __init__(self, version, variant, h, w, c, win, input, expected):
        self.version = version
        self.variant = variant
        self.h, self.w, self.c, self.win = h, w, c, win
        self.input = input          # float32 [c][h][w]
        self.expected = expected    # float32 [c][h][w]

    @staticmethod
    def load(path):
        """fixture.rs:37-80. Raises ValueError naming the file and what is wrong."""
        path = str(path)
        try:
            with open(path, "rb") as f:
                b = f.read()
        except OSError as e:
            raise ValueError(f"{path}: {e}") from None
        if len(b) < 40 or b[:4] != MAGIC:
            raise ValueError(f"{path}: not a scunet fixture (want 4-byte magic SCUF)")
        version, h, w, c, win, vlen = struct.unpack_from("<6I", b, 4)
        if version != 1:
            raise ValueError(f"{path}: fixture version {version}, this engine reads 1")
        if len(b) < 28 + vlen:
            raise ValueError(f"{path}: the variant string claims {vlen} bytes, the file is shorter")
        try:
            variant = b[28:28 + vlen].decode("utf-8")
        except UnicodeDecodeError as e:
            raise ValueError(f"{path}: variant is not utf-8: {e}") from None
        off = 28 + vlen
        n = h * w * c
        need = off + 4 * 2 * n
        if len(b) != need:
            raise ValueError(f"{path}: {need} bytes expected for {h}x{w}x{c} in and out, {len(b)} present")
        x = np.frombuffer(b, dtype="<f4", count=n, offset=off).astype(np.float32).reshape(c, h, w)
        y = np.frombuffer(b, dtype="<f4", count=n, offset=off + 4 * n).astype(np.float32).reshape(c, h, w)
        return Fixture(version, variant, h, w, c, win, x, y)

    def compare(self, got):
        """(worst |diff|, its flat NCHW index, mean |diff|) against the expected output."""
        got = np.asarray(got, np.float32).ravel()
        want = self.expected.ravel()
        if got.shape != want.shape:
            raise ValueError("backend returned the wrong number of pixels")
        d = np.abs(want - got)
        at = int(d.argmax())
        return float(d[at]), at, float(d.astype(np.float64).mean())

    def locate(self, idx):
        """A flat NCHW index as (y, x, channel)."""
        plane = self.h * self.w
        c, rem = divmod(int(idx), plane)
        return rem // self.w, rem % self.w, c


def save(path, x, y, variant, win=8):
    """Write `x` (the input) and `y` (the expected output), both [c][h][w] or [1][c][h][w],
    as a version-1 fixture (the container tools/make_fixture.py:48-56 writes)."""
    x = np.asarray(x, np.float32)
    y = np.asarray(y, np.float32)
    if x.ndim == 4:
        x = x[0]
    if y.ndim == 4:
        y = y[0]
    if x.shape != y.shape or x.ndim != 3:
        raise ValueError(f"input {x.shape} and output {y.shape} must be the same [c][h][w]")
    c, h, w = x.shape
    v = variant.encode("utf-8")
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<6I", 1, h, w, c, win, len(v)))
        f.write(v)
        f.write(np.ascontiguousarray(x, "<f4").tobytes())
        f.write(np.ascontiguousarray(y, "<f4").tobytes())
