"""Helpers of the stage-replay parity tests: a device stage is compared with
the oracle's primitive applied to the device's own inputs of that stage, so
differences cannot accumulate over stages and the bars can be stated in bf16
steps."""
import numpy as np


def bf16_order(values) -> np.ndarray:
    """Monotone integer of each bf16 value (float32 holding bf16 bits): one
    apart for neighbouring bf16 values, +0 and -0 both 0."""
    bits = (np.ascontiguousarray(values, np.float32).view(np.uint32) >> 16).astype(np.int64)
    mag = bits & 0x7FFF
    return np.where(bits & 0x8000, -mag, mag)


def bf16_steps(a, b) -> np.ndarray:
    """How many bf16 values apart a and b are, elementwise."""
    return np.abs(bf16_order(a) - bf16_order(b))


def stage_report(dev, ref):
    """(fraction of identical elements, largest distance in bf16 steps)."""
    s = bf16_steps(dev, ref)
    return float(np.mean(s == 0)), int(s.max()) if s.size else 0


def bf16_spacing(values) -> np.ndarray:
    """The distance from each bf16 value to the next one away from zero
    (2^(e - 7) for a normal value of exponent e; 2^-133 below the normal
    range; 0 for zero)."""
    v = np.abs(np.asarray(values, np.float64))
    e = np.floor(np.log2(np.where(v > 0, v, 1.0)))
    sp = np.exp2(np.maximum(e, -126.0) - 7.0)
    return np.where(v > 0, sp, 0.0)


def projection_bound(x, w, b=None) -> np.ndarray:
    """Largest |y_dev - y_ref| for two bf16-rounded fp32 sums of the same
    products x w^T (+ b) in different orders: each sum within
    (K + 1) 2^-24 sum|x w| of the exact value, then half a bf16 step of
    its own rounding (added by the caller from the two results)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    s = np.abs(x) @ np.abs(w).T
    if b is not None:
        s = s + np.abs(np.asarray(b, np.float64))[None, :]
    return 2.0 * (x.shape[1] + 1) * 2.0 ** -24 * s


def projection_close(dev, ref, x, w, b=None, min_identical: float = 0.9):
    """(ok, identical fraction, worst |dev - ref| / allowed)."""
    dev = np.asarray(dev, np.float64)
    ref = np.asarray(ref, np.float64)
    allowed = projection_bound(x, w, b) + 0.5 * (bf16_spacing(dev) + bf16_spacing(ref))
    excess = np.abs(dev - ref) / np.maximum(allowed, 1e-300)
    same = float(np.mean(dev == ref))
    worst = float(excess.max()) if excess.size else 0.0
    return same >= min_identical and worst <= 1.0, same, worst
