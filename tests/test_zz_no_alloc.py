"""scunet_hip_run_device_noalloc: the forward with its scratch in the library's static device
array (no hipMalloc/hipFree in the call) gives the same bits as scunet_hip_run_device, on two
calls in a row, the second with a smaller image (the array keeps the first call's contents),
and refuses an image whose scratch exceeds the array without touching the device."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _device_run(be, x, noalloc):
    c, h, w = x.shape
    xp = be.malloc(x.nbytes)
    yp = be.malloc(x.nbytes)
    try:
        be.h2d(xp, x)
        if noalloc:
            be.run_device_noalloc(xp, c, h, w, yp)
        else:
            be.run_device(xp, c, h, w, yp)
        return be.d2h(np.empty_like(x), yp)
    finally:
        be.free(xp)
        be.free(yp)


def test_noalloc_forward_equals_run_device(weights_path):
    from scunet_hip import Hip, synth
    big = synth.noisy_image(71, 3, 300, 260, 25)      # pads to 320x320
    small = synth.noisy_image(72, 3, 72, 100, 25)     # pads to 128x128
    with Hip(weights_path) as be:
        want_big = _device_run(be, big, False)
        want_small = _device_run(be, small, False)
        scratch_before = be.footprint()[1]
        for _ in range(2):
            got_big = _device_run(be, big, True)
            got_small = _device_run(be, small, True)
            assert np.array_equal(got_big, want_big)
            assert np.array_equal(got_small, want_small)
        assert np.isfinite(got_big).all()
        # The arena of the allocating path is neither used nor grown by the no-alloc calls.
        assert be.footprint()[1] == scratch_before


def test_noalloc_fp16_mode_equals_run_device(weights_path):
    from scunet_hip import Hip, synth
    x = synth.noisy_image(73, 3, 128, 192, 25)
    with Hip(weights_path) as be:
        be.set_precision("fp16")
        assert np.array_equal(_device_run(be, x, True), _device_run(be, x, False))


def test_noalloc_refuses_an_image_beyond_the_static_scratch(weights_path):
    from scunet_hip import BackendError, Hip
    with Hip(weights_path) as be:
        xp = be.malloc(1 << 20)
        yp = be.malloc(1 << 20)
        try:
            # 512x512 needs 400 MiB of scratch; the static array holds 256 MiB. The input
            # buffer is far smaller than the claimed image: the refusal comes before any launch.
            with pytest.raises(BackendError, match=r"needs \d+ bytes of scratch; the static scratch holds 268435456"):
                be.run_device_noalloc(xp, 3, 512, 512, yp)
        finally:
            be.free(xp)
            be.free(yp)
