"""GPU: the device packer is bit-exact with the oracle, and the backend
seam's sticky loss and fault injection behave as internal/driver requires
(plan.go:385-391; cpu.go:179-191)."""
import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import F16, F32, U32, workloads

pytestmark = pytest.mark.gpu


def device_quantize(dev, w):
    n = w.size
    wb = dev.upload(np.ascontiguousarray(w, np.float32).ravel())
    pb = dev.alloc(((n + 7) // 8,), U32)
    sb = dev.alloc(((n + 127) // 128,), F16)
    zb = dev.alloc(((n + 127) // 128,), F16)
    pb.write(np.full((n + 7) // 8, 0xDEADBEEF, np.uint32))  # must be overwritten
    dev.int4_quantize(wb, n, pb, sb, zb)
    out = pb.numpy(), sb.numpy(), zb.numpy()
    for b in (wb, pb, sb, zb):
        b.free()
    return out


@pytest.mark.parametrize("kind", ["normal", "far", "tiny", "denorm", "huge", "ties",
                                  "signed_zero", "nan_inf", "nan_first", "halves",
                                  "near_halves"])
@pytest.mark.parametrize("n", [1, 9, 128, 129, 1000, 8192 + 5])
def test_device_packer_is_bit_exact(dev, kind, n):
    rng = np.random.default_rng(n + len(kind))
    gens = {
        "normal": lambda: rng.standard_normal(n) * 0.02,
        "far": lambda: 1000 + rng.random(n),
        "tiny": lambda: rng.standard_normal(n) * 1e-7,
        "denorm": lambda: rng.standard_normal(n) * 1e-40,
        "huge": lambda: rng.standard_normal(n) * 1e30,
        "ties": lambda: np.round(rng.standard_normal(n) * 8) / 8,
        "signed_zero": lambda: np.where(rng.random(n) < 0.5, -0.0, 0.0),
        "nan_inf": lambda: np.where(rng.random(n) < 0.03, np.nan,
                                    np.where(rng.random(n) < 0.03, np.inf,
                                             rng.standard_normal(n))),
        "nan_first": lambda: np.where(np.arange(n) % 128 == 0, np.nan, rng.standard_normal(n)),
        # groups spanning 0..15 quantize with s = 1, z = 0: every weight an
        # exact tie of the round-half-to-even rule
        "halves": lambda: rng.integers(0, 31, n) / 2.0,
        # and weights a few ulps to 2^-10 off those ties
        "near_halves": lambda: (rng.integers(0, 31, n) / 2.0) *
        (1 + rng.choice([-1.0, 1.0], n) * 2.0 ** -rng.integers(10, 24, n)),
    }
    w = np.asarray(gens[kind](), np.float32)
    got = device_quantize(dev, w)
    want = oracle.int4_quantize(w)
    for g, x, what in zip(got, want, ("codes", "scales", "zeros")):
        assert np.array_equal(g, x), what


def test_device_packer_at_the_decode_shape(dev):
    rng = np.random.Generator(np.random.PCG64(1))
    w = (rng.standard_normal((4096, 14336)) * 0.02).astype(np.float32)
    got = device_quantize(dev, w)
    want = accel_amd.int4_quantize(w)
    for g, x in zip(got, want):
        assert np.array_equal(g, x)


def test_injected_loss_is_sticky_and_reported(dev):
    L = workloads.linear(1, 256, 256, seed=2)
    w = dev.upload_int4(L.packed, L.scales, L.zeros, L.K * L.N)
    a = dev.upload(L.x[0])
    out = dev.alloc((L.N,), F32)
    try:
        dev.inject_loss(2)
        dev.Int4MatVec(a, w, out)          # submission 1: runs
        dev.sync()
        with pytest.raises(accel_amd.DeviceLost):
            dev.Int4MatVec(a, w, out)      # submission 2: lost, launches nothing
        assert dev.lost
        with pytest.raises(accel_amd.DeviceLost):
            dev.Int4MatVec(a, w, out)      # and stays lost
        with pytest.raises(accel_amd.DeviceLost):
            dev.sync()
        e = dev.event()
        assert dev.event_done(e)           # a lost device is done
    finally:
        # reopen: a fresh device state for the tests that follow
        dev.close()
        accel_amd.Device(dev.index)
    assert not dev.lost
    dev.Int4MatVec(a, w, out)
    dev.sync()
    for b in (a, out):
        b.free()
    w.free()
