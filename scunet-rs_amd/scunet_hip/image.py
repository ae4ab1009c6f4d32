"""PNG in, PNG out (src/image.rs:17-69 of the reference) over the library's codec
(``scunet_image_read`` / ``scunet_image_write``, declared in include/scunet_image.h).

The contract is the reference's: 8-bit samples, ``value / 255`` as float32 ``[c][h][w]``;
RGB and RGBA read as three channels (alpha dropped), gray and gray+alpha as one; writing
clamps to [0, 1] and stores ``(u8)(v * 255 + 0.5)``. Palette images fail with
"unsupported colour type Indexed" (image.rs:31). Failures raise :class:`ImageError`
carrying the library's message, the ``Err(String)`` of image.rs.
"""
import ctypes

import numpy as np

from . import load_library

__all__ = ["Image", "ImageError", "read", "write"]

_sz = ctypes.c_size_t
_f = ctypes.POINTER(ctypes.c_float)


class ImageError(ValueError):
    """A PNG that could not be read or written."""


class Image:
    """image.rs:9-15: ``data`` is float32 ``[c][h][w]`` in [0, 1]."""

    def __init__(self, c, h, w, data):
        self.c, self.h, self.w, self.data = c, h, w, data


def _lib():
    L = load_library()
    if not getattr(L, "_image_declared", False):
        L.scunet_image_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(_f), ctypes.POINTER(_sz),
                                        ctypes.POINTER(_sz), ctypes.POINTER(_sz)]
        L.scunet_image_free.argtypes = [_f]
        L.scunet_image_free.restype = None
        L.scunet_image_write.argtypes = [ctypes.c_char_p, _f, _sz, _sz, _sz]
        L.scunet_image_error.restype = ctypes.c_char_p
        L._image_declared = True
    return L


def read(path):
    """image.rs:17-43."""
    L = _lib()
    p, c, h, w = _f(), _sz(), _sz(), _sz()
    if L.scunet_image_read(str(path).encode(), ctypes.byref(p), ctypes.byref(c), ctypes.byref(h),
                           ctypes.byref(w)) != 0:
        raise ImageError(L.scunet_image_error().decode())
    try:
        n = c.value * h.value * w.value
        data = np.ctypeslib.as_array(p, shape=(n,)).copy().reshape(c.value, h.value, w.value)
    finally:
        L.scunet_image_free(p)
    return Image(c.value, h.value, w.value, data)


def write(path, data, c=None, h=None, w=None):
    """image.rs:45-69: ``data`` is ``[c][h][w]`` (or flat with c, h, w given)."""
    L = _lib()
    a = np.ascontiguousarray(data, dtype=np.float32)
    if c is None:
        c, h, w = a.shape
    if a.size != c * h * w:
        raise ImageError(f"{a.size} values for a {c}x{h}x{w} image")
    if L.scunet_image_write(str(path).encode(), a.ctypes.data_as(_f), c, h, w) != 0:
        raise ImageError(L.scunet_image_error().decode())
