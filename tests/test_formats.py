"""Packed formats and host quantizers of lowbit_amd (CPU only).

Two kinds of checks:

* known answers, held as data tables below. Each table cites where its values
  come from: the reference's format definitions (src/lowbit/formats.py) and the
  values its format tests pin (tests/test_formats.py of the reference);
* properties of the quantizers over seeded random inputs. These are the
  half-step error bound, padding that decodes to zero, and the shared-exponent
  rule. The packers are also checked against the oracle's independent unpacker
  and quantizer.
"""
import numpy as np
import pytest

from lowbit_amd import formats as F
from oracle import reference as O

ROWS = 6


def _codes_of(index_map, packed):
    """Codes read back from `packed` through an explicit (byte, shift) map."""
    byte, shift = index_map
    return (packed[:, byte] >> shift) & 15


def _nibble_map(kp, block):
    """Closed form of the packed layout: element e of a row sits in byte
    (e // block) * block/2 + (e % block) % (block/2), low nibble for the first
    half of its block and high nibble for the second (src/lowbit/csrc/lowbit.h:9-19)."""
    e = np.arange(kp)
    half = block // 2
    byte = (e // block) * half + (e % block) % half
    shift = np.where((e % block) >= half, 4, 0)
    return byte, shift


# ------------------------------------------------------------------ nibble layout

@pytest.mark.parametrize("block,nblocks", [(32, 1), (32, 5), (128, 1), (128, 3)])
def test_packed_layout_follows_closed_form(rng, block, nblocks):
    kp = block * nblocks
    codes = rng.integers(0, 16, size=(ROWS, kp), dtype=np.uint8)
    packed = F.pack_nibbles(codes, block)
    assert packed.shape == (ROWS, kp // 2) and packed.dtype == np.uint8
    np.testing.assert_array_equal(_codes_of(_nibble_map(kp, block), packed), codes)
    # inverse, and the oracle's own unpacker
    np.testing.assert_array_equal(F.unpack_nibbles(packed, block), codes)
    np.testing.assert_array_equal(O.unpack_codes(packed, block), codes)


def test_single_code_lands_in_one_nibble():
    for block, elem, byte, high in [(128, 133, 69, False), (128, 197, 69, True), (32, 50, 18, True)]:
        codes = np.zeros((1, 2 * block), np.uint8)
        codes[0, elem] = 9
        packed = F.pack_nibbles(codes, block)
        assert np.flatnonzero(packed[0]).tolist() == [byte]
        assert packed[0, byte] == (9 << 4 if high else 9)


# ------------------------------------------------------------------ int4 group 128: known answers

# (name, weights of one 128-element group, asym, scale rule, expected scale, expected zero,
#  expected codes or None). Values follow the quantizer's closed form
# (src/lowbit/formats.py:90-142): sym s = max|w| / 7 and q = rint(w / s) + 8;
# asym s = (max - min) / 15, z = rint(-min / s); a zero scale becomes 1.
_G = 128
INT4_KATS = [
    ("zero group, sym", np.zeros(_G), False, "absmax", 1.0, 8, np.full(_G, 8)),
    ("zero group, asym", np.zeros(_G), True, "absmax", 1.0, 0, np.zeros(_G)),
    ("constant 5, sym", np.full(_G, 5.0), False, "absmax", np.float32(5.0) / np.float32(7.0), 8, np.full(_G, 15)),
    ("constant 5, asym", np.full(_G, 5.0), True, "absmax", np.float32(5.0) / np.float32(15.0), 0, np.full(_G, 15)),
    ("ramp -1.5..3, asym", np.linspace(-1.5, 3.0, _G), True, "absmax",
     np.float32(4.5) / np.float32(15.0), 5, None),
    ("on-grid step 0.25, sym", np.resize(np.arange(-7, 8), _G) * 0.25, False, "absmax", 0.25, 8,
     np.resize(np.arange(-7, 8), _G) + 8),
    ("signed max -4, sym", np.resize([-4.0, 1.0, 2.0, -1.0], _G), False, "signed-max", 0.5, 8,
     np.resize([0, 10, 12, 6], _G)),
]


@pytest.mark.parametrize("name,w,asym,rule,scale,zero,codes", INT4_KATS, ids=[k[0] for k in INT4_KATS])
def test_int4_known_answers(name, w, asym, rule, scale, zero, codes):
    q = F.quantize_int4(np.asarray(w, np.float32)[None], asym=asym, scale=rule)
    assert q.scales[0, 0] == np.float32(scale)
    assert (8 if q.zeros is None else int(q.zeros[0, 0])) == zero
    if codes is not None:
        np.testing.assert_array_equal(q.codes()[0], codes)
    if name.startswith("ramp"):
        c = q.codes()[0]
        assert (c[0], c[-1]) == (0, 15)  # min and max land on the ends of the code range


def test_int4_on_grid_weights_are_reproduced_exactly(rng):
    # every group holds +-7 steps, so max|w| / 7 is exactly the step (reference pins
    # the same fact, tests/test_formats.py:55-64)
    steps = rng.integers(-7, 8, size=(4, 2 * _G))
    steps[:, [0, _G]] = [7, -7]
    w = (steps * np.float32(0.25)).astype(np.float32)
    q = F.quantize_int4(w)
    np.testing.assert_array_equal(q.scales, np.float32(0.25))
    np.testing.assert_array_equal(q.dequantize(), w)


def test_int4_rejects_unknown_rules():
    w = np.ones((1, 8), np.float32)
    for kwargs in ({"asym": True, "scale": "signed-max"}, {"scale": "bogus"}):
        with pytest.raises(ValueError):
            F.quantize_int4(w, **kwargs)


# ------------------------------------------------------------------ int4: properties

@pytest.mark.parametrize("k", [1, 127, 128, 257, 300])
@pytest.mark.parametrize("asym", [False, True])
def test_int4_properties(rng, k, asym):
    w = (rng.standard_normal((ROWS, k)) * 3).astype(np.float32)
    q = F.quantize_int4(w, asym=asym)
    kp = q.kp
    assert kp % _G == 0 and kp - _G < k <= kp
    codes = q.codes()
    assert codes.shape == (ROWS, kp) and codes.max() <= 15
    step = np.repeat(q.scales, _G, axis=1)[:, :k]
    err = np.abs(q.dequantize() - w)
    assert np.all(err <= 0.5 * step * (1 + 1e-5) + 1e-7)  # round to nearest: half a step
    # the padding decodes to exactly 0: its code is the group's zero-point
    z = np.full((ROWS, 1), 8) if q.zeros is None else q.zeros[:, -1:]
    assert np.all(codes[:, k:] == z)
    # byte-identical with the oracle's decode of the same arrays
    np.testing.assert_array_equal(O.dequant_int4(q.qw, q.scales, q.zeros, k).astype(np.float32), q.dequantize())


@pytest.mark.parametrize("k", [1, 128, 300])
def test_int4_signed_max_properties(rng, k):
    w = (rng.standard_normal((9, k)) * 3).astype(np.float32)
    q = F.quantize_int4(w, scale="signed-max")
    err = np.abs(q.dequantize() - w)
    step = np.abs(np.repeat(q.scales, _G, axis=1)[:, :k])
    # the element of largest magnitude in the first group is code 0 and exact
    g0 = w[:, :min(k, _G)]
    i = np.argmax(np.abs(g0), axis=1)
    r = np.arange(9)
    assert np.all(q.codes()[r, i] == 0)
    np.testing.assert_allclose(q.dequantize()[r, i], g0[r, i], rtol=1e-6)
    # at most one step everywhere (values near -m clip from +8 to +7), half a step
    # nearly everywhere, and no worse on average than the absmax rule
    assert np.all(err <= step * (1 + 1e-5) + 1e-7)
    assert np.mean(err <= 0.5 * step * (1 + 1e-5) + 1e-7) > 0.95
    assert np.mean(err ** 2) <= np.mean((F.quantize_int4(w).dequantize() - w) ** 2)


# ------------------------------------------------------------------ E2M1 / E8M0: known answers

# (input, decoded value): the E2M1 grid maps to itself; ties go to the even code; the
# range saturates at +-6; -0 and tiny negatives give the canonical +0 code
# (src/lowbit/formats.py:23-24,182-194; the reference pins the ties and the
# saturation in tests/test_formats.py:75-91).
E2M1_KATS = ([(v, v) for v in F.E2M1_VALUES.tolist()] +
             [(0.25, 0.0), (0.75, 1.0), (1.25, 1.0), (1.75, 2.0), (2.5, 2.0), (3.5, 4.0), (5.0, 4.0),
              (-0.25, 0.0), (-0.75, -1.0), (-1.25, -1.0), (-1.75, -2.0), (-2.5, -2.0), (-3.5, -4.0),
              (-5.0, -4.0), (7.9, 6.0), (-100.0, -6.0), (0.3, 0.5), (2.6, 3.0)])


def test_e2m1_encode_known_answers():
    x = np.array([a for a, _ in E2M1_KATS], np.float32)
    want = np.array([b for _, b in E2M1_KATS], np.float32)
    np.testing.assert_array_equal(F.E2M1_VALUES[F.fp32_to_e2m1(x)], want)
    np.testing.assert_array_equal(F.fp32_to_e2m1(np.array([-0.0, -0.1], np.float32)), [0, 0])


# (byte, value) of the E8M0 decode: 2^(e - 127), 0 -> the float32 subnormal 2^-127,
# 255 -> NaN (src/lowbit/formats.py:175-179, src/lowbit/csrc/lowbit.h:84-92; the
# reference pins these bytes in tests/test_formats.py:94-99)
E8M0_KATS = [(0, 2.0 ** -127), (1, 2.0 ** -126), (126, 0.5), (127, 1.0), (128, 2.0), (200, 2.0 ** 73),
             (254, 2.0 ** 127)]


def test_e8m0_decode_known_answers():
    e = np.array([b for b, _ in E8M0_KATS] + [255], np.uint8)
    f = F.e8m0_to_float(e)
    np.testing.assert_array_equal(f[:-1], np.array([v for _, v in E8M0_KATS], np.float32))
    assert np.isnan(f[-1])
    assert int(f[0].view(np.uint32)) == 0x00400000


# ------------------------------------------------------------------ MXFP4: properties and grid

@pytest.mark.parametrize("k", [32, 100, 4096])
def test_mxfp4_properties(rng, k):
    w = rng.standard_normal((ROWS, k)).astype(np.float32)
    q = F.quantize_mxfp4(w)
    assert q.kp % 32 == 0 and q.kp - 32 < k <= q.kp
    # shared exponent of every block: floor(log2(amax)) - 2
    blocks = np.zeros((ROWS, q.kp), np.float32)
    blocks[:, :k] = w
    amax = np.abs(blocks.reshape(ROWS, -1, 32)).max(axis=2)
    np.testing.assert_array_equal(q.e8m0.astype(np.int64) - 127, np.floor(np.log2(amax)).astype(np.int64) - 2)
    # the widest E2M1 step is 2 (4 -> 6), so no value is off by more than 2 scales
    scale = np.repeat(F.e8m0_to_float(q.e8m0), 32, axis=1)[:, :k]
    assert np.all(np.abs(q.dequantize() - w) <= 2.0 * scale)
    np.testing.assert_array_equal(O.dequant_mxfp4(q.qw, q.e8m0, k).astype(np.float32), q.dequantize())


def test_mxfp4_grid_values_times_four_are_exact(rng):
    # block maximum 6 * 4 = 24: floor(log2 24) - 2 = 2, E8M0 byte 129 (the reference pins
    # the same case, tests/test_formats.py:115-123)
    codes = rng.integers(0, 16, size=(3, 64)).astype(np.uint8)
    codes[:, [0, 32]] = 7
    w = (F.E2M1_VALUES[codes] * np.float32(4.0)).astype(np.float32)
    q = F.quantize_mxfp4(w)
    assert np.all(q.e8m0 == 129)
    np.testing.assert_array_equal(q.dequantize(), w)


# ------------------------------------------------------------------ per-token int8 activations

@pytest.mark.parametrize("m,k", [(1, 1), (4, 200), (3, 1000)])
def test_act_quant_properties(rng, m, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    a = F.quantize_act_int8(x)
    kp = F.pad_to(k, _G)
    assert a.xq.shape == (m, kp) and a.gsum.shape == (m, kp // _G)
    assert np.all(a.xq[:, k:] == 0) and np.abs(a.xq.astype(np.int32)).max() <= 127
    np.testing.assert_array_equal(a.gsum, a.xq.astype(np.int32).reshape(m, -1, _G).sum(axis=2))
    assert np.all(np.abs(a.dequantize()[:, :k] - x) <= 0.5 * a.scale[:, None] * (1 + 1e-6))


def test_act_quant_matches_oracle(rng):
    x = (rng.standard_normal((5, 1000)) * 3).astype(np.float32)
    x[2] = 0
    a = F.quantize_act_int8(x)
    xq, xs, asum = O.quant_act_int8(x)
    np.testing.assert_array_equal(a.xq, xq)
    np.testing.assert_array_equal(a.scale, xs)
    np.testing.assert_array_equal(a.gsum, asum)


# ------------------------------------------------------------------ effective weight bytes

def test_nbytes_is_the_metric_byte_count():
    # packed codes + fp32 scales (+ uint8 zero-points) or + E8M0 (src/lowbit/formats.py:76-77,163-164)
    n, k = 11008, 4096
    assert F.quantize_int4(np.ones((8, k), np.float32), asym=True).nbytes == 8 * (k // 2 + (k // 128) * 5)
    assert F.quantize_int4(np.ones((8, k), np.float32)).nbytes == 8 * (k // 2 + (k // 128) * 4)
    assert F.quantize_mxfp4(np.ones((8, k), np.float32)).nbytes == 8 * (k // 2 + k // 32)
    assert n * (k // 2 + (k // 128) * 5) == 24_305_664
    assert n * (k // 2 + k // 32) == 23_953_408
