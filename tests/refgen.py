"""Input generators of the reference's own GEMV differential tests
(gemv.rs:693-730), restated so the same vectors can be regenerated here.

xrng is xorshift64 (shifts 13/7/17); rscales/rinput do their arithmetic in
f32 as the Rust code does, and round to f16 with round-to-nearest-even
(half::f16::from_f32).
"""
import numpy as np

from qtts.synth import Q4

M64 = (1 << 64) - 1


class XRng:
    def __init__(self, seed):
        self.s = seed & M64

    def next(self):
        s = self.s
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        self.s = s
        return s


def rvec(st, n, mag):
    """rvec of the reference's conv tests (conv.rs:707-711):
    ((xrng % 2000) as f32 / 1000 - 1) * mag, in f32."""
    r = np.fromiter((st.next() % 2000 for _ in range(n)), dtype=np.float32, count=n)
    return (r / np.float32(1000.0) - np.float32(1.0)) * np.float32(mag)


def rbytes(st, n):
    return np.array([st.next() & 0xFF for _ in range(n)], dtype=np.uint8)


def rscales(st, n, zero_frac):
    out = np.empty(n, np.float16)
    for i in range(n):
        r = (st.next() % 1000) / 1000.0
        if r < zero_frac:
            out[i] = np.float16(0.0)
        else:
            v = (np.float32(st.next() % 2000) / np.float32(1000.0) - np.float32(1.0)) * np.float32(0.05)
            out[i] = np.float16(v)
    return out.view(np.uint16)


def rinput(st, n, zero_frac):
    out = np.empty(n, np.float32)
    for i in range(n):
        r = (st.next() % 1000) / 1000.0
        if r < zero_frac:
            out[i] = 0.0
        else:
            out[i] = (np.float32(st.next() % 2000) / np.float32(1000.0) - np.float32(1.0)) * np.float32(2.0)
    return out


def case(k, n, seed, in_zero=0.0, sc_zero=0.0):
    """check_case (gemv.rs:735-754): (x, Q4 weight)."""
    st = XRng(seed)
    groups = n // 32
    packed = rbytes(st, k * groups * 16).reshape(k, groups * 16)
    scales = rscales(st, k * groups, sc_zero).reshape(k, groups)
    x = rinput(st, k, in_zero)
    return x, Q4(packed, scales, k, n)


# The reference's differential cases (gemv.rs:756-861).
SHAPE_CASES = [(64, 2048, 1), (64, 6144, 2), (32, 1024, 3), (16, 256, 4), (1, 32, 5)]
SPARSE_CASES = [(48, 1024, 11, 0.3, 0.2), (32, 2048, 12, 0.5, 0.5)]
