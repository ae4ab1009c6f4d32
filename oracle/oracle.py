"""TEST INFRASTRUCTURE - the CPU oracle's Python face. Not part of the product.

ctypes bindings for ``build/libscunet_oracle.so``, the C++ restatement of the
reference's ``src/cpu.rs``. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may import this module.

Parity status of each function (how the restatement is pinned, see tests/):
  conv3x3 / conv2x2s2 / conv1x1 / conv_t2x2  brute-force definitions on small inputs and
                                             torch.nn.functional (library) results
  layer_norm                                 closed form
  erf / gelu                                 math.erf (|d| < 1.5e-7, the A&S bound)
  rel_pos_table                              upstream's cord/relation construction
  mask_hit                                   brute-force rebuild of upstream's 4 slice rules
  attention                                  the reference's two known-answer tests + a
                                             brute-force per-window numpy evaluation
  pad / crop                                 closed form + the reference's plan asserts
  trans_block / conv_trans_block / forward   golden vectors written by tools/reference.py
                                             (tests/golden/make_golden.py)
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libscunet_oracle.so")

_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t
HOOK = ctypes.CFUNCTYPE(None, ctypes.c_char_p, _f, ctypes.c_size_t, ctypes.c_void_p)


class _OW(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int),
        ("names", ctypes.POINTER(ctypes.c_char_p)),
        ("ptrs", ctypes.POINTER(_f)),
        ("numel", ctypes.POINTER(ctypes.c_size_t)),
        ("in_nc", ctypes.c_int),
        ("dim", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("window", ctypes.c_int),
        ("config", ctypes.c_int * 7),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_erf.restype = ctypes.c_double
        L.oracle_erf.argtypes = [ctypes.c_double]
        L.oracle_mask_hit.restype = ctypes.c_int
        L.oracle_mask_hit.argtypes = [_sz] * 7
        L.oracle_get_threads.restype = ctypes.c_int
        L.oracle_forward_dump.argtypes = [ctypes.POINTER(_OW), _f, _sz, _sz, _f, HOOK, ctypes.c_void_p]
        L.oracle_conv_trans_block.argtypes = [ctypes.POINTER(_OW), ctypes.c_char_p, _f, _sz, _sz, _sz,
                                              _f, _f, _f, _f, _f, _f]
        L.oracle_forward_dump.restype = ctypes.c_int
        L.oracle_conv_trans_block.restype = ctypes.c_int
        L.oracle_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f)


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib().oracle_last_error().decode())


def set_threads(n):
    lib().oracle_set_threads(int(n))


def threads():
    return lib().oracle_get_threads()


class Weights:
    """A checkpoint as the oracle sees it: name -> float32 array, plus the architecture."""

    def __init__(self, tensors, meta):
        self.t = {k: _c32(v) for k, v in tensors.items()}
        self.meta = meta
        self.in_nc = int(meta["in_nc"])
        self.dim = int(meta["dim"])
        self.head_dim = int(meta["head_dim"])
        self.window = int(meta["window_size"])
        self.config = [int(v) for v in str(meta["config"]).split(",")]
        names = list(self.t)
        self._names = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
        self._ptrs = (_f * len(names))(*[_p(self.t[n]) for n in names])
        self._numel = (ctypes.c_size_t * len(names))(*[self.t[n].size for n in names])
        self.ow = _OW(len(names), self._names, self._ptrs, self._numel, self.in_nc, self.dim,
                      self.head_dim, self.window, (ctypes.c_int * 7)(*self.config))

    @classmethod
    def load(cls, path):
        import sys
        sys.path.insert(0, os.path.join(_HERE, "..", "scunet-rs_amd"))
        from scunet_hip.safetensors_io import read_safetensors
        t, meta = read_safetensors(path)
        return cls(t, meta)

    def block_dims(self, prefix):
        total = self.t[f"{prefix}.conv1_1.weight"].shape[0]
        trans = self.t[f"{prefix}.trans_block.msa.linear.weight"].shape[0]
        return total - trans, trans


def conv3x3(x, wt):
    c_in, h, w = x.shape
    c_out = wt.shape[0]
    out = np.empty((c_out, h, w), np.float32)
    lib().oracle_conv3x3(_p(_c32(x)), _sz(c_in), _sz(c_out), _sz(h), _sz(w), _p(_c32(wt)), _p(out))
    return out


def conv2x2s2(x, wt):
    c_in, h, w = x.shape
    c_out = wt.shape[0]
    out = np.empty((c_out, h // 2, w // 2), np.float32)
    lib().oracle_conv2x2s2(_p(_c32(x)), _sz(c_in), _sz(c_out), _sz(h), _sz(w), _p(_c32(wt)), _p(out))
    return out


def conv1x1(x, wt, bias=None):
    c_in = x.shape[0]
    n = x[0].size
    c_out = wt.shape[0]
    out = np.empty((c_out,) + x.shape[1:], np.float32)
    lib().oracle_conv1x1(_p(_c32(x)), _sz(c_in), _sz(c_out), _sz(n), _p(_c32(wt)),
                         _p(_c32(bias)) if bias is not None else None, _p(out))
    return out


def conv_t2x2(x, wt):
    c_in, h, w = x.shape
    c_out = wt.shape[1]
    out = np.empty((c_out, 2 * h, 2 * w), np.float32)
    lib().oracle_conv_t2x2(_p(_c32(x)), _sz(c_in), _sz(c_out), _sz(h), _sz(w), _p(_c32(wt)), _p(out))
    return out


def layer_norm(x, wg, bs):
    c = x.shape[-1]
    rows = x.size // c
    out = np.empty_like(_c32(x))
    lib().oracle_layer_norm(_p(_c32(x)), _sz(rows), _sz(c), _p(_c32(wg)), _p(_c32(bs)), _p(out))
    return out


def gelu(x):
    y = _c32(x).copy()
    lib().oracle_gelu_inplace(_p(y), _sz(y.size))
    return y


def erf(x):
    return lib().oracle_erf(float(x))


def mask_hit(p, t, wh, ww, nwh, nww, win):
    return bool(lib().oracle_mask_hit(p, t, wh, ww, nwh, nww, win))


def rel_pos_table(params, win):
    out = np.empty((win * win, win * win), np.float32)
    lib().oracle_rel_pos_table(_p(_c32(params)), _sz(win), _p(out))
    return out


def attention(x_hwc, h, w, c, win, shift, emb_w, emb_b, lin_w, lin_b, rp):
    """cpu.rs:602-758 on a [h][w][c] token plane -> [h][w][c]."""
    heads = rp.shape[0]
    out = np.empty((h * w * c,), np.float32)
    lib().oracle_attention(_p(_c32(x_hwc)), _sz(h), _sz(w), _sz(c), _sz(win), _sz(shift),
                           _p(_c32(emb_w)), _p(_c32(emb_b)), _p(_c32(lin_w)), _p(_c32(lin_b)),
                           _p(_c32(rp)), _sz(heads), _p(out))
    return out.reshape(h * w, c)


def pad_replicate(x, hp, wp):
    c, h, w = x.shape
    out = np.empty((c, hp, wp), np.float32)
    lib().oracle_pad_replicate(_p(_c32(x)), _sz(c), _sz(h), _sz(w), _sz(hp), _sz(wp), _p(out))
    return out


def crop(x, h, w):
    c, hp, wp = x.shape
    out = np.empty((c, h, w), np.float32)
    lib().oracle_crop(_p(_c32(x)), _sz(c), _sz(h), _sz(w), _sz(hp), _sz(wp), _p(out))
    return out


def trans_block(wt, prefix, x_hwc, h, w, shift, want_msa=False):
    """cpu.rs:782-861 for block `prefix` on a [h*w][c] token plane."""
    tp = prefix + ".trans_block"
    g = lambda k: wt.t[f"{tp}.{k}"]
    c = g("ln1.weight").shape[0]
    rp = g("msa.relative_position_params")
    out = np.empty((h * w, c), np.float32)
    msa = np.empty((h * w, c), np.float32) if want_msa else None
    lib().oracle_trans_block(
        _p(_c32(x_hwc)), _sz(h), _sz(w), _sz(c), _sz(wt.window), _sz(shift),
        _p(g("ln1.weight")), _p(g("ln1.bias")), _p(g("msa.embedding_layer.weight")),
        _p(g("msa.embedding_layer.bias")), _p(g("msa.linear.weight")), _p(g("msa.linear.bias")),
        _p(rp), _sz(rp.shape[0]), _p(g("ln2.weight")), _p(g("ln2.bias")), _p(g("mlp.0.weight")),
        _p(g("mlp.0.bias")), _p(g("mlp.2.weight")), _p(g("mlp.2.bias")), _p(out), _p(msa))
    return (out, msa) if want_msa else out


def conv_trans_block(wt, prefix, x, shift, dump=False):
    """cpu.rs:976-983 on a [c][h][w] plane; with dump, also the block's interior planes."""
    c, h, w = x.shape
    conv, trans = wt.block_dims(prefix)
    out = np.empty_like(_c32(x))
    d = None
    if dump:
        d = dict(expand=np.empty((c, h, w), np.float32), conv_half=np.empty((conv, h, w), np.float32),
                 trans_half=np.empty((trans, h, w), np.float32),
                 msa=np.empty((h * w, trans), np.float32), res=np.empty((c, h, w), np.float32))
    args = [_p(d[k]) if d else None for k in ("expand", "conv_half", "trans_half", "msa", "res")]
    _check(lib().oracle_conv_trans_block(ctypes.byref(wt.ow), prefix.encode(), _p(_c32(x)), _sz(h), _sz(w),
                                         _sz(shift), _p(out), *args))
    return (out, d) if dump else out


def forward_dump(wt, x_padded, keep=None):
    """cpu.rs:1175-1321 -> (output [in_nc][hp][wp], {stage name: plane copy})."""
    c, hp, wp = x_padded.shape
    out = np.empty((c, hp, wp), np.float32)
    stages = {}

    def hook(name, ptr, n, _user):
        nm = name.decode()
        if keep is None or nm in keep:
            stages[nm] = np.ctypeslib.as_array(ptr, shape=(n,)).copy()

    cb = HOOK(hook)
    _check(lib().oracle_forward_dump(ctypes.byref(wt.ow), _p(_c32(x_padded)), _sz(hp), _sz(wp), _p(out), cb,
                                     None))
    return out, stages


def forward(wt, x_padded):
    return forward_dump(wt, x_padded, keep=())[0]


PAD_TO = 64


def plan(h, w):
    """plan.rs:43-47: the padded geometry, ceil to a multiple of 64 on each axis."""
    return (h + PAD_TO - 1) // PAD_TO * PAD_TO, (w + PAD_TO - 1) // PAD_TO * PAD_TO


def run(wt, x):
    """backend.rs:63-105 on the CPU path: pad, forward, crop."""
    c, h, w = x.shape
    hp, wp = plan(h, w)
    xp = _c32(x) if (hp, wp) == (h, w) else pad_replicate(x, hp, wp)
    y = forward(wt, xp)
    return crop(y, h, w) if (hp, wp) != (h, w) else y
