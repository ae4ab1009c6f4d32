"""Host-side mirror of the reference crate's backend interface over libscunet_hip.so.

The reference (jacobsparts/scunet-rs) exposes its devices through ``trait Backend``
(src/backend.rs:19-56), ``backend::run`` (backend.rs:63-105) and ``Plan``
(src/plan.rs:26-118). :class:`Hip` is that trait for the MI355X library, with the same
method names, argument meanings and error behaviour (a failed call raises
:class:`BackendError` carrying the library's message, the ``Err(String)`` of the
reference); :func:`run` and :class:`Plan` are the free functions and geometry.

There is no fallback: if the shared library is missing, or the machine has no HIP
device, constructing :class:`Hip` raises.
"""
import ctypes
import os

import numpy as np

__all__ = ["Hip", "Plan", "run", "BackendError", "LIB_PATH", "load_library", "PAD_TO", "check_min_size"]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "..", "lib", "libscunet_hip.so")

# The symbols include/scunet_hip.h declares.
EXPORTS = [
    "scunet_hip_create", "scunet_hip_create_from_tensors", "scunet_hip_create_error", "scunet_hip_destroy", "scunet_hip_last_error",
    "scunet_hip_name", "scunet_hip_arch", "scunet_hip_variant", "scunet_hip_set_precision", "scunet_hip_precision",
    "scunet_hip_forward", "scunet_hip_forward_device",
    "scunet_hip_forward_dump", "scunet_hip_run", "scunet_hip_run_device", "scunet_hip_run_device_noalloc",
    "scunet_hip_run_batch",
    "scunet_hip_device_need", "scunet_hip_footprint",
    "scunet_hip_release_scratch", "scunet_hip_synchronize", "scunet_hip_stream", "scunet_hip_profile",
    "scunet_hip_profile_report", "scunet_hip_malloc", "scunet_hip_free", "scunet_hip_h2d", "scunet_hip_d2h",
    "scunet_hip_copy",
    "scunet_hip_block_probe", "scunet_hip_op_probe", "scunet_hip_linear_probe",
    "scunet_hip_layer_norm_probe", "scunet_hip_attention_kernel_probe", "scunet_hip_gather_probe",
    "scunet_hip_window_round_trip", "scunet_hip_attention_probe", "scunet_hip_bench_attn",
]

_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
HOOK = ctypes.CFUNCTYPE(None, ctypes.c_char_p, _f, ctypes.c_size_t, ctypes.c_void_p)
# scunet_hip_tensor_lookup: (user, name, shape[8], ndim) -> data pointer or NULL.
LOOKUP = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(_sz),
                          ctypes.POINTER(_sz))


class ArchInfo(ctypes.Structure):
    """scunet_hip_arch_info: the fields of the reference's Weights (weights.rs:83-97)."""
    _fields_ = [("variant", ctypes.c_char_p), ("in_nc", _sz), ("dim", _sz), ("head_dim", _sz),
                ("window", _sz), ("config", _sz * 7)]


class BackendError(RuntimeError):
    """A failed backend call: the reference's ``Err(String)``."""


_lib = None


def load_library(path=None):
    """Load libscunet_hip.so and declare its signatures. Raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = os.path.abspath(path or LIB_PATH)
    if not os.path.exists(p):
        raise BackendError(f"{p} is not built (run `make -C scunet-rs_amd` or __graft_entry__.build())")
    L = ctypes.CDLL(p)
    L.scunet_hip_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp)]
    L.scunet_hip_create_error.restype = ctypes.c_char_p
    L.scunet_hip_create_from_tensors.argtypes = [ctypes.POINTER(ArchInfo), LOOKUP, _vp, ctypes.POINTER(_vp)]
    L.scunet_hip_destroy.argtypes = [_vp]
    L.scunet_hip_last_error.argtypes = [_vp]
    L.scunet_hip_last_error.restype = ctypes.c_char_p
    L.scunet_hip_name.argtypes = [_vp]
    L.scunet_hip_name.restype = ctypes.c_char_p
    ip = ctypes.POINTER(ctypes.c_int)
    L.scunet_hip_arch.argtypes = [_vp, ip, ip, ip, ip, ip]
    L.scunet_hip_variant.argtypes = [_vp]
    L.scunet_hip_variant.restype = ctypes.c_char_p
    L.scunet_hip_set_precision.argtypes = [_vp, ctypes.c_int]
    L.scunet_hip_precision.argtypes = [_vp]
    L.scunet_hip_forward.argtypes = [_vp, _f, _sz, _sz, _sz, _f]
    L.scunet_hip_forward_device.argtypes = [_vp, _vp, _sz, _sz, _sz, _vp]
    L.scunet_hip_forward_dump.argtypes = [_vp, _f, _sz, _sz, _sz, _f, HOOK, _vp]
    L.scunet_hip_run.argtypes = [_vp, _f, _sz, _sz, _sz, _f]
    L.scunet_hip_run_device.argtypes = [_vp, _vp, _sz, _sz, _sz, _vp]
    L.scunet_hip_run_device_noalloc.argtypes = [_vp, _vp, _sz, _sz, _sz, _vp]
    L.scunet_hip_run_batch.argtypes = [_vp, _f, _sz, _sz, _sz, _sz, _f]
    L.scunet_hip_device_need.argtypes = [_vp, _sz, _sz, _sz, ctypes.c_int, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]
    L.scunet_hip_footprint.argtypes = [_vp, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]
    L.scunet_hip_release_scratch.argtypes = [_vp]
    L.scunet_hip_synchronize.argtypes = [_vp]
    L.scunet_hip_stream.argtypes = [_vp]
    L.scunet_hip_stream.restype = _vp
    L.scunet_hip_profile.argtypes = [_vp, ctypes.c_int]
    L.scunet_hip_profile_report.argtypes = [_vp, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_long),
                                            ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double), ctypes.c_int, ip]
    L.scunet_hip_malloc.argtypes = [_vp, ctypes.POINTER(_vp), _sz]
    L.scunet_hip_free.argtypes = [_vp, _vp]
    L.scunet_hip_h2d.argtypes = [_vp, _vp, _vp, _sz]
    L.scunet_hip_d2h.argtypes = [_vp, _vp, _vp, _sz]
    L.scunet_hip_copy.argtypes = [_vp, _vp, _vp, _sz]
    L.scunet_hip_block_probe.argtypes = [_vp, ctypes.c_char_p, _sz, _sz, _sz, _f, _f]
    L.scunet_hip_op_probe.argtypes = [_vp, ctypes.c_char_p, ctypes.c_char_p, _f, _sz, _sz, _sz, _sz, _f]
    L.scunet_hip_linear_probe.argtypes = [_vp, ctypes.c_char_p, _f, _sz, _sz, _sz, _f]
    L.scunet_hip_layer_norm_probe.argtypes = [_vp, ctypes.c_char_p, _f, _sz, _sz, _f]
    L.scunet_hip_attention_kernel_probe.argtypes = [_vp, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f, _f]
    L.scunet_hip_gather_probe.argtypes = [_vp, _sz, _sz, _sz, _sz, _f, _f]
    L.scunet_hip_window_round_trip.argtypes = [_vp, _sz, _sz, _sz, _sz, _f, _f]
    L.scunet_hip_attention_probe.argtypes = [_vp, ctypes.c_char_p, _sz, _sz, _sz, _sz, _f, _f]
    L.scunet_hip_bench_attn.argtypes = [_vp, _vp, _f, _vp, _sz, _sz, _sz, _sz, _sz, ctypes.c_int,
                                        ctypes.POINTER(ctypes.c_double)]
    if path is None:
        _lib = L
    return L


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return a.ctypes.data_as(_f)


# ---------------------------------------------------------------------------
# Plan (src/plan.rs)
# ---------------------------------------------------------------------------

PAD_TO = 64   # plan.rs:40: three stride-2 stages times the 8-pixel window


class Plan:
    """plan.rs:26-57: the padded geometry of one image."""

    def __init__(self, h, w, win=8):
        self.h, self.w, self.win = int(h), int(w), int(win)
        self.hp = -(-self.h // PAD_TO) * PAD_TO
        self.wp = -(-self.w // PAD_TO) * PAD_TO

    def plane(self):
        return self.hp * self.wp

    def windows(self, dn):
        return ((self.hp >> dn) // self.win, (self.wp >> dn) // self.win)

    def __repr__(self):
        return f"Plan(h={self.h}, w={self.w}, hp={self.hp}, wp={self.wp}, win={self.win})"


def check_min_size(h, w, win=8):
    """plan.rs:105-118. Raises BackendError like the reference returns Err."""
    p = Plan(h, w, win)
    if p.hp < 8 * win or p.wp < 8 * win:
        raise BackendError(
            f"{h}x{w} pads to {p.hp}x{p.wp}, but the 1/8-resolution body needs at least "
            f"{win}x{win} pixels there - i.e. {8 * win}x{8 * win} before padding.")


def pad_replicate(x, hp, wp):
    """plan.rs:67-82 on the host (the device path fuses it into m_head)."""
    c, h, w = x.shape
    return np.pad(x, ((0, 0), (0, hp - h), (0, wp - w)), mode="edge")


def crop(y, h, w):
    """plan.rs:85-94."""
    return np.ascontiguousarray(y[:, :h, :w])


# ---------------------------------------------------------------------------
# The backend (src/backend.rs:19-56)
# ---------------------------------------------------------------------------

class Hip:
    """``impl Backend`` for the MI355X library. Construction mirrors ``Cuda::new``
    (src/cuda.rs:192-241) over ``Weights::load`` (src/weights.rs:101-185)."""

    def __init__(self, weights_path=None, lib_path=None, *, tensors=None, arch=None):
        """From a safetensors file (``weights_path``), or, like ``Cuda::new(&Weights)``, from
        tensors the caller already holds: ``tensors`` maps names to float32 arrays and
        ``arch`` gives variant, in_nc, dim, head_dim, window and config
        (scunet_hip_create_from_tensors)."""
        self._lib = load_library(lib_path)
        h = _vp()
        if tensors is not None:
            rc = self._create_from_tensors(tensors, arch, h)
        else:
            rc = self._lib.scunet_hip_create(os.fsencode(weights_path), ctypes.byref(h))
        if rc != 0:
            raise BackendError(self._lib.scunet_hip_create_error().decode())
        self._h = h
        a = [ctypes.c_int() for _ in range(4)]
        cfg = (ctypes.c_int * 7)()
        self._lib.scunet_hip_arch(h, *[ctypes.byref(v) for v in a], cfg)
        self.in_nc, self.dim, self.head_dim, self.window = (v.value for v in a)
        self.config = list(cfg)
        self.variant = self._lib.scunet_hip_variant(h).decode()

    def _create_from_tensors(self, tensors, arch, h):
        held = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in tensors.items()}

        def lookup(_user, name, shape, ndim):
            a = held.get(name.decode())
            if a is None:
                return None
            if a.ndim > 8:
                ndim[0] = a.ndim
                return a.ctypes.data
            for i, e in enumerate(a.shape):
                shape[i] = e
            ndim[0] = a.ndim
            return a.ctypes.data

        cb = LOOKUP(lookup)
        info = ArchInfo(str(arch["variant"]).encode(), int(arch["in_nc"]), int(arch["dim"]),
                        int(arch["head_dim"]), int(arch["window"]), (_sz * 7)(*[int(v) for v in arch["config"]]))
        return self._lib.scunet_hip_create_from_tensors(ctypes.byref(info), cb, None, ctypes.byref(h))

    # -- lifetime --
    def close(self):
        if getattr(self, "_h", None):
            self._lib.scunet_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc != 0:
            raise BackendError(self._lib.scunet_hip_last_error(self._h).decode())

    # -- trait Backend --
    def name(self):
        return self._lib.scunet_hip_name(self._h).decode()

    # -- arithmetic mode (no counterpart in the reference) --
    PRECISIONS = {"fp32": 0, "fp16": 1, "fp32_mfma": 2}

    def set_precision(self, mode):
        """"fp32" (the reference's arithmetic to fp32 rounding, the default: split-operand
        products on the bf16 matrix cores where a kernel has them), "fp32_mfma" (every
        product on the fp32 matrix cores) or "fp16" (fp16 MFMA operands, fp32 accumulation
        and planes)."""
        self._check(self._lib.scunet_hip_set_precision(self._h, self.PRECISIONS[mode]))

    def precision(self):
        m = self._lib.scunet_hip_precision(self._h)
        return {v: k for k, v in self.PRECISIONS.items()}[m]

    def forward(self, x, plan):
        """backend.rs:23-25: padded [c][hp][wp] in, a fresh [c][hp][wp] out."""
        x = _c32(x)
        if x.shape != (self.in_nc, plan.hp, plan.wp):
            raise BackendError(f"expected {self.in_nc * plan.hp * plan.wp} floats ({self.in_nc} channels of "
                               f"{plan.hp}x{plan.wp}), got {x.size}")
        y = np.empty_like(x)
        self._check(self._lib.scunet_hip_forward(self._h, _p(x), x.shape[0], plan.hp, plan.wp, _p(y)))
        return y

    def forward_dump(self, x, hook):
        """cpu.rs:1175-1321's stage hook over the device walker: hook(name, nchw_plane)."""
        x = _c32(x)
        c, hp, wp = x.shape
        y = np.empty_like(x)

        def cb(name, ptr, n, _u):
            hook(name.decode(), np.ctypeslib.as_array(ptr, shape=(n,)).copy())

        fn = HOOK(cb)
        self._check(self._lib.scunet_hip_forward_dump(self._h, _p(x), c, hp, wp, _p(y), fn, None))
        return y

    def footprint(self):
        w, s = _sz(), _sz()
        self._lib.scunet_hip_footprint(self._h, ctypes.byref(w), ctypes.byref(s))
        return (w.value, s.value)

    def profile_report(self):
        rows = self.profile_rows()
        total = sum(r[2] for r in rows)
        print(f"  ---- device time per kernel (total {total:.1f} ms) ----")
        for name, n, ms, _f1, _b in rows:
            print(f"  {ms:9.1f} ms  {n:6} launches  {name}")

    def mem_report(self):
        w, s = self.footprint()
        print(f"  ---- device memory: {w / 2**20:.1f} MiB weights, {s / 2**20:.1f} MiB scratch ----")

    def release_scratch(self):
        self._check(self._lib.scunet_hip_release_scratch(self._h))

    # -- profiling (cuda.rs:106-135 SCUNET_PROFILE) --
    def profile(self, on=True):
        self._check(self._lib.scunet_hip_profile(self._h, 1 if on else 0))

    def profile_rows(self, cap=64):
        names = (ctypes.c_char_p * cap)()
        launches = (ctypes.c_long * cap)()
        ms, flop, byts = ((ctypes.c_double * cap)() for _ in range(3))
        n = ctypes.c_int()
        self._check(self._lib.scunet_hip_profile_report(self._h, names, launches, ms, flop, byts, cap,
                                                        ctypes.byref(n)))
        return [(names[i].decode(), launches[i], ms[i], flop[i], byts[i]) for i in range(min(n.value, cap))]

    # -- device-resident entry points (device pointers as ints) --
    def malloc(self, nbytes):
        p = _vp()
        self._check(self._lib.scunet_hip_malloc(self._h, ctypes.byref(p), nbytes))
        return p.value

    def free(self, ptr):
        self._check(self._lib.scunet_hip_free(self._h, _vp(ptr)))

    def h2d(self, ptr, arr):
        arr = np.ascontiguousarray(arr)
        self._check(self._lib.scunet_hip_h2d(self._h, _vp(ptr), arr.ctypes.data_as(_vp), arr.nbytes))

    def d2h(self, arr, ptr):
        self._check(self._lib.scunet_hip_d2h(self._h, arr.ctypes.data_as(_vp), _vp(ptr), arr.nbytes))
        return arr

    def copy(self, dst, src, nbytes):
        """A plain device copy kernel (the traffic-counter calibration kernel)."""
        self._check(self._lib.scunet_hip_copy(self._h, _vp(dst), _vp(src), nbytes))

    def forward_device(self, xptr, c, hp, wp, yptr):
        self._check(self._lib.scunet_hip_forward_device(self._h, _vp(xptr), c, hp, wp, _vp(yptr)))

    def run_device(self, xptr, c, h, w, yptr):
        self._check(self._lib.scunet_hip_run_device(self._h, _vp(xptr), c, h, w, _vp(yptr)))

    def run_device_noalloc(self, xptr, c, h, w, yptr):
        """run_device with the forward's scratch in the library's static device array
        (scunet_hip_run_device_noalloc): no device allocation in the call."""
        self._check(self._lib.scunet_hip_run_device_noalloc(self._h, _vp(xptr), c, h, w, _vp(yptr)))

    def synchronize(self):
        self._check(self._lib.scunet_hip_synchronize(self._h))

    def run_fused(self, x):
        """backend::run with the pad and crop on the device (scunet_hip_run)."""
        x = _c32(x)
        c, h, w = x.shape
        y = np.empty_like(x)
        self._check(self._lib.scunet_hip_run(self._h, _p(x), c, h, w, _p(y)))
        return y

    def run_batch(self, x):
        """n images of one size, [n][c][h][w]: one upload, n forwards, one download."""
        x = _c32(x)
        n, c, h, w = x.shape
        y = np.empty_like(x)
        self._check(self._lib.scunet_hip_run_batch(self._h, _p(x), n, c, h, w, _p(y)))
        return y

    def device_need(self, h, w, host_io=True):
        """(scratch bytes after an h x w forward, bytes not held yet): memguard's device_need."""
        tot, more = _sz(), _sz()
        self._check(self._lib.scunet_hip_device_need(self._h, self.in_nc, h, w, int(host_io),
                                                     ctypes.byref(tot), ctypes.byref(more)))
        return tot.value, more.value

    # -- probes (cuda.rs:1153-1597) --
    def block_dump(self, prefix, h, w, shift, x):
        x = _c32(x)
        out = np.empty_like(x)
        self._check(self._lib.scunet_hip_block_probe(self._h, prefix.encode(), h, w, shift, _p(x), _p(out)))
        return out

    def op_probe(self, which, name, x, c_in, c_out, h, w):
        x = _c32(x)
        n = {"conv2x2s2": (h // 2) * (w // 2), "conv_t2x2": 4 * h * w}.get(which, h * w)
        out = np.empty(c_out * n, np.float32)
        self._check(self._lib.scunet_hip_op_probe(self._h, which.encode(), name.encode(), _p(x), c_in, c_out,
                                                  h, w, _p(out)))
        return out

    def linear_probe(self, name, x, rows, c_in, c_out):
        x = _c32(x)
        out = np.empty(rows * c_out, np.float32)
        self._check(self._lib.scunet_hip_linear_probe(self._h, name.encode(), _p(x), rows, c_in, c_out, _p(out)))
        return out

    def layer_norm_probe(self, name, x, rows, c):
        x = _c32(x)
        out = np.empty(rows * c, np.float32)
        self._check(self._lib.scunet_hip_layer_norm_probe(self._h, name.encode(), _p(x), rows, c, _p(out)))
        return out

    def attention_kernel_probe(self, h, w, c, heads, hd, shift, qkv, rp):
        qkv, rp = _c32(qkv), _c32(rp)
        out = np.empty((h // 8) * (w // 8) * 64 * c, np.float32)
        self._check(self._lib.scunet_hip_attention_kernel_probe(self._h, h, w, c, heads, hd, shift, _p(qkv),
                                                                _p(rp), _p(out)))
        return out

    def gather_probe(self, h, w, c, shift, x):
        x = _c32(x)
        out = np.empty(h * w * c, np.float32)
        self._check(self._lib.scunet_hip_gather_probe(self._h, h, w, c, shift, _p(x), _p(out)))
        return out

    def window_round_trip(self, h, w, c, shift, x):
        x = _c32(x)
        out = np.empty_like(x)
        self._check(self._lib.scunet_hip_window_round_trip(self._h, h, w, c, shift, _p(x), _p(out)))
        return out

    def attention_probe(self, prefix, h, w, c, shift, x):
        x = _c32(x)
        out = np.empty(h * w * c, np.float32)
        self._check(self._lib.scunet_hip_attention_probe(self._h, prefix.encode(), h, w, c, shift, _p(x), _p(out)))
        return out

    def bench_attn(self, qkv_ptr, rp, out_ptr, nwh, nww, c, heads, shift, iters):
        rp = _c32(rp)
        ms = ctypes.c_double()
        self._check(self._lib.scunet_hip_bench_attn(self._h, _vp(qkv_ptr), _p(rp), _vp(out_ptr), nwh, nww, c,
                                                    heads, shift, iters, ctypes.byref(ms)))
        return ms.value


def run(be, x, c=None, h=None, w=None):
    """backend.rs:63-105: replicate-pad to ceil64, forward, check the length, crop."""
    x = _c32(x)
    c, h, w = x.shape if c is None else (c, h, w)
    plan = Plan(h, w, getattr(be, "window", 8))
    check_min_size(h, w, plan.win)
    padded = x if (plan.hp, plan.wp) == (h, w) else _c32(pad_replicate(x, plan.hp, plan.wp))
    y = be.forward(padded, plan)
    if y.size != c * plan.plane():
        raise BackendError(f"{be.name()}: the backend returned {y.size} floats for a {plan.hp}x{plan.wp} "
                           f"plane of {c} channels")
    y = y.reshape(c, plan.hp, plan.wp)
    return crop(y, h, w) if (plan.hp, plan.wp) != (h, w) else y
