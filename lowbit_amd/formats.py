"""Packed low-bit weight formats and the host-side quantizers (numpy, one-time work).

These are the public data layouts of the drop-in API. The GEMMs never see dense
weights: they read the packed bytes below straight from HBM.

Shapes follow nn.Linear: W is [N, K] (N outputs, K inputs) and every GEMM
computes Y[M, N] = X[M, K] @ W^T. K is padded to Kp, a multiple of the block
(128 for int4, 32 for MXFP4); padded weight codes decode to exactly 0 and the
GEMMs see zero-padded X, so padding never changes a result.

Layouts (row n of W occupies Kp/2 contiguous bytes):
  int4, group 128  group g is bytes [64g, 64g+64) of the row; byte j holds
                   element 128g+j in its low nibble and element 128g+64+j in
                   its high nibble. value = (q - z) * s, q in 0..15, s fp32,
                   z uint8 (8 when ``zeros is None``).
  int4, group 32   (an extension: the reference ships group 128 only) the same
                   "j / j+half" rule per group of 32: group g is bytes
                   [16g, 16g+16), byte j holds 32g+j and 32g+16+j.
  MXFP4, block 32  block b is bytes [16b, 16b+16); byte j holds element 32b+j
                   (low nibble) and 32b+16+j (high nibble). Codes are OCP E2M1
                   (sign | 2-bit exponent | 1-bit mantissa), value =
                   e2m1(q) * 2^(e8m0[n, b] - 127).

The layouts, the quantization rules and their float32 operation order restate
the reference's format module (src/lowbit/formats.py:19-248) so that the same
inputs give the same bytes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GROUP = 128   # int4 group size (elements)
GROUPS = (128, 32)  # supported int4 group sizes
MXBLOCK = 32  # MXFP4 block size (elements)

# OCP MX E2M1: code -> value. Bit 3 is the sign, bits 2..1 the exponent, bit 0
# the mantissa (src/lowbit/formats.py:23-24).
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
E2M1_EMAX = 2  # exponent of the largest E2M1 normal (6 = 1.5 * 2^2)


def pad_to(k: int, block: int) -> int:
    """Smallest multiple of ``block`` that is >= k."""
    return ((k + block - 1) // block) * block


# ------------------------------------------------------------------ nibble packing

def pack_nibbles(codes: np.ndarray, block: int) -> np.ndarray:
    """Pack uint8 codes [N, Kp] (0..15) into bytes [N, Kp/2], "j / j+half" per block.

    Restates src/lowbit/formats.py:34-44: inside each block, byte j carries
    element j (low nibble) and element j + block/2 (high nibble).
    """
    n, kp = codes.shape
    if kp % block:
        raise ValueError(f"row length {kp} is not a multiple of the block {block}")
    half = block // 2
    blocks = np.asarray(codes, dtype=np.uint8).reshape(n, kp // block, 2, half)
    low, high = blocks[:, :, 0, :], blocks[:, :, 1, :]
    return np.bitwise_or(low, np.left_shift(high, 4)).reshape(n, kp // 2)


def unpack_nibbles(packed: np.ndarray, block: int) -> np.ndarray:
    """Inverse of :func:`pack_nibbles`: bytes [N, Kp/2] -> codes [N, Kp]."""
    n, nbytes = packed.shape
    half = block // 2
    p = np.asarray(packed, dtype=np.uint8).reshape(n, (2 * nbytes) // block, 1, half)
    return np.concatenate([p & 0x0F, p >> 4], axis=2).reshape(n, 2 * nbytes)


# ------------------------------------------------------------------ int4, group 128

@dataclass
class Int4Weights:
    """int4 weights, group 128 (or 32), fp32 scale per group, optional uint8 zero-point.

    value[n, k] = (q[n, k] - z[n, k // group]) * s[n, k // group], z = 8 when
    symmetric (src/lowbit/formats.py:56-87; `group` = 32 is this package's extension).
    """
    qw: np.ndarray            # uint8 [N, Kp/2] packed codes
    scales: np.ndarray        # float32 [N, G]
    zeros: np.ndarray | None  # uint8 [N, G], or None (symmetric, z = 8)
    k: int                    # logical K (before padding)
    group: int = GROUP        # elements per group: 128 (the reference's) or 32

    @property
    def n(self) -> int:
        return self.qw.shape[0]

    @property
    def kp(self) -> int:
        return self.qw.shape[1] * 2

    @property
    def nbytes(self) -> int:
        """Effective weight bytes: codes + scales (+ zeros). The GB/s metric divides this."""
        extra = 0 if self.zeros is None else self.zeros.nbytes
        return self.qw.nbytes + self.scales.nbytes + extra

    def codes(self) -> np.ndarray:
        return unpack_nibbles(self.qw, self.group)

    def dequantize(self) -> np.ndarray:
        """Dense float32 [N, K] (for baselines and checks only; the GEMMs never do this)."""
        g = self.kp // self.group
        q = self.codes().astype(np.float32).reshape(self.n, g, self.group)
        if self.zeros is None:
            z = np.float32(8.0)
        else:
            z = self.zeros.astype(np.float32)[:, :, None]
        dense = (q - z) * self.scales[:, :, None]
        return dense.reshape(self.n, self.kp)[:, : self.k]


def quantize_int4(w: np.ndarray, asym: bool = False, scale: str = "absmax", group: int = GROUP) -> Int4Weights:
    """Round-to-nearest int4 with group size 128 (src/lowbit/formats.py:90-142), or 32
    (`group=32`: the same rules per group of 32, packed "j / j+half" per group).

    absmax (symmetric):  s = absmax / 7,               q = clip(rint(w/s), -8, 7) + 8
    signed-max:          s = m / -8 (m = the element of largest magnitude, sign kept);
                         the extreme element lands on code 0, s may be negative
    asymmetric:          s = (max(w,0) - min(w,0)) / 15, z = clip(rint(-min/s), 0, 15),
                         q = clip(rint(w/s) + z, 0, 15)
    A zero scale becomes 1. Padded positions get code z, so they decode to 0.
    """
    if scale not in ("absmax", "signed-max"):
        raise ValueError(f"scale must be 'absmax' or 'signed-max', not {scale!r}")
    if asym and scale != "absmax":
        raise ValueError("scale='signed-max' is a symmetric rule (asym=False)")
    if group not in GROUPS:
        raise ValueError(f"group must be one of {GROUPS}, not {group!r}")
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    kp = pad_to(k, group)
    ng = kp // group
    padded = np.zeros((n, kp), np.float32)
    padded[:, :k] = w
    grp = padded.reshape(n, ng, group)
    real = (np.arange(kp) < k).reshape(1, ng, group)
    one = np.float32(1.0)
    if asym:
        # Padding is +0 and the range is clamped to include 0 anyway, so the zero
        # padding can take part in the max/min without changing either.
        hi = np.maximum(grp.max(axis=2), np.float32(0.0))
        lo = np.minimum(grp.min(axis=2), np.float32(0.0))
        s = ((hi - lo) / np.float32(15)).astype(np.float32)
        s = np.where(s > 0, s, one).astype(np.float32)
        z = np.clip(np.rint(-lo / s), 0, 15).astype(np.uint8)
        zc = z[:, :, None]
        q = np.clip(np.rint(grp / s[:, :, None]) + zc, 0, 15)
        q = np.where(real, q, zc)
        zeros = z
    else:
        if scale == "signed-max":
            pick = np.abs(grp).argmax(axis=2)[:, :, None]
            m = np.take_along_axis(grp, pick, axis=2)[:, :, 0]
            s = (m / np.float32(-8)).astype(np.float32)
            s = np.where(s != 0, s, one).astype(np.float32)
        else:
            s = (np.abs(grp).max(axis=2) / np.float32(7)).astype(np.float32)
            s = np.where(s > 0, s, one).astype(np.float32)
        q = np.clip(np.rint(grp / s[:, :, None]), -8, 7) + 8
        q = np.where(real, q, 8)
        zeros = None
    codes = q.astype(np.uint8).reshape(n, kp)
    return Int4Weights(pack_nibbles(codes, group), s.astype(np.float32), zeros, k, group)


# ------------------------------------------------------------------ MXFP4

@dataclass
class MXFP4Weights:
    """OCP MXFP4: E2M1 elements in blocks of 32 sharing an E8M0 scale 2^(e-127)
    (src/lowbit/formats.py:147-172)."""
    qw: np.ndarray    # uint8 [N, Kp/2] packed E2M1 codes
    e8m0: np.ndarray  # uint8 [N, Kp/32] biased exponents
    k: int

    @property
    def n(self) -> int:
        return self.qw.shape[0]

    @property
    def kp(self) -> int:
        return self.qw.shape[1] * 2

    @property
    def nbytes(self) -> int:
        return self.qw.nbytes + self.e8m0.nbytes

    def codes(self) -> np.ndarray:
        return unpack_nibbles(self.qw, MXBLOCK)

    def dequantize(self) -> np.ndarray:
        vals = E2M1_VALUES[self.codes()].reshape(self.n, -1, MXBLOCK)
        dense = vals * e8m0_to_float(self.e8m0)[:, :, None]
        return dense.reshape(self.n, self.kp)[:, : self.k]


def e8m0_to_float(e: np.ndarray) -> np.ndarray:
    """E8M0 -> float32: 2^(e-127); e = 0 is the subnormal 2^-127, e = 255 is NaN
    (src/lowbit/formats.py:175-179, src/lowbit/csrc/lowbit.h:84-88)."""
    e = np.asarray(e, dtype=np.uint8)
    nan = e == 255
    out = np.ldexp(np.float32(1.0), np.where(nan, 0, e.astype(np.int32) - 127)).astype(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def fp32_to_e2m1(v: np.ndarray) -> np.ndarray:
    """Round float32 (already divided by the block scale) to E2M1 codes.

    Round to nearest with ties to the even mantissa code, saturating at +-6
    (src/lowbit/formats.py:182-194). The magnitude code is the number of
    decision points below |v|: ties at .25, 1.25, 2.5, 5 round down and ties
    at .75, 1.75, 3.5 round up. -0 and values that round to 0 give code 0.
    """
    v = np.asarray(v, np.float32)
    a = np.abs(v)
    mag = np.zeros(a.shape, np.uint8)
    for edge, inclusive in ((0.25, False), (0.75, True), (1.25, False), (1.75, True),
                            (2.5, False), (3.5, True), (5.0, False)):
        mag += (a >= edge) if inclusive else (a > edge)
    negative = np.signbit(v) & (mag > 0)
    return (mag | (negative.astype(np.uint8) << 3)).astype(np.uint8)


def quantize_mxfp4(w: np.ndarray) -> MXFP4Weights:
    """OCP MX v1.0: shared exponent floor(log2(amax)) - 2 per block of 32
    (src/lowbit/formats.py:197-212). The exponent is taken with numpy's float32
    log2, as the reference does, so the bytes match for the same input."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    kp = pad_to(k, MXBLOCK)
    padded = np.zeros((n, kp), np.float32)
    padded[:, :k] = w
    blk = padded.reshape(n, kp // MXBLOCK, MXBLOCK)
    amax = np.abs(blk).max(axis=2)
    nonzero = amax > 0
    with np.errstate(divide="ignore"):
        lg = np.log2(amax, where=nonzero, out=np.zeros_like(amax))
    shared = np.where(nonzero, np.floor(lg) - E2M1_EMAX, 0)
    e = np.clip(shared + 127, 0, 254).astype(np.uint8)
    codes = fp32_to_e2m1(blk / e8m0_to_float(e)[:, :, None]).reshape(n, kp)
    return MXFP4Weights(pack_nibbles(codes, MXBLOCK), e, k)


# ------------------------------------------------------------------ activations

@dataclass
class Int8Acts:
    """Per-token symmetric int8 activations (src/lowbit/formats.py:217-224)."""
    xq: np.ndarray     # int8 [M, Kp]
    scale: np.ndarray  # float32 [M]
    gsum: np.ndarray   # int32 [M, Kp/128], per-group sum of the codes

    def dequantize(self) -> np.ndarray:
        return self.xq.astype(np.float32) * self.scale[:, None]


def pad_acts(x: np.ndarray, kp: int) -> np.ndarray:
    """float32, C-contiguous [M, kp] copy of x with zero columns appended (no copy if
    it already is one) (src/lowbit/formats.py:227-233)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape[1] == kp:
        return x
    out = np.zeros((x.shape[0], kp), np.float32)
    out[:, : x.shape[1]] = x
    return out


def quantize_act_int8(x: np.ndarray, kp: int | None = None) -> Int8Acts:
    """Per-token int8: s = absmax/127 (1 for an all-zero row), q = clip(rint(x/s), +-127).

    Host twin of the device quantizer that runs inside every W4A8 GEMM; both
    give identical bytes (src/lowbit/formats.py:236-248, src/lowbit/csrc/dispatch.c:231-257).
    """
    x = np.asarray(x, np.float32)
    kp = pad_to(x.shape[1], GROUP) if kp is None else kp
    xp = pad_acts(x, kp)
    amax = np.abs(xp).max(axis=1)
    s = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(xp / s[:, None]), -127, 127).astype(np.int8)
    gsum = q.reshape(q.shape[0], -1, GROUP).astype(np.int32).sum(axis=2).astype(np.int32)
    return Int8Acts(q, s, gsum)
