"""OCP FP8 e4m3fn and bf16 number formats, restated from their bit layouts.

Test infrastructure only (see ``oracle/__init__.py``).

e4m3fn (the gfx950 FP8 format: ``using fp8e4m3 = __hip_fp8_e4m3`` at
``include/cdna4/common/base_types.cuh:45``, with 1.0 encoded as 0x38 at
``base_types.cuh:163``): 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits,
no infinities, S.1111.111 is NaN, largest finite 448 (0x7E).

Encoding rule frozen for this path: round to nearest, ties to even, saturate
finite overflow to +-448 and map NaN to 0x7F/0xFF.  That is HIP's
``__HIP_SATFINITE`` conversion used by the reference's ``convertor<fp8e4m3,
float>`` (``base_types.cuh:423-432``); ``torch.float8_e4m3fn`` agrees below
448 and is the library routine the tests pin this against.

bf16: round to nearest even from fp32 (``v_cvt_pk_bf16_f32`` semantics,
``base_types.cuh:350-358``).  The reference's scalar bf16 store truncates
(``base_types.cuh:334-343``); this path specifies RNE for every bf16 output.
"""
import numpy as np

E4M3_MAX = 448.0


def _build_decode_lut():
    lut = np.empty(256, dtype=np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            lut[code] = np.nan
        elif e == 0:
            lut[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            lut[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return lut


E4M3_LUT = _build_decode_lut()
# positive finite values in code order 0x00..0x7E; strictly increasing
_POS_VALS = E4M3_LUT[:0x7F].astype(np.float64)


def e4m3_to_f32(q):
    """Decode e4m3fn bytes (uint8 array) to float32."""
    q = np.asarray(q, dtype=np.uint8)
    return E4M3_LUT[q]


def f32_to_e4m3(x):
    """Encode float32 to e4m3fn bytes: RNE, saturating, NaN -> 0x7F|sign.

    Implemented as a nearest-value search over the 127 positive finite codes
    (ties -> the even code, i.e. mantissa LSB 0), independent of the bit-trick
    encoder the HIP kernels use.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    nan = np.isnan(a)
    a = np.where(nan, 0.0, a)
    hi = np.searchsorted(_POS_VALS, a, side="left")  # first value >= a
    hi = np.minimum(hi, 0x7E)
    lo = np.maximum(hi - 1, 0)
    dhi = _POS_VALS[hi] - a
    dlo = a - _POS_VALS[lo]
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a >= E4M3_MAX, 0x7E, code)
    code = np.where(a == 0.0, 0, code)
    code = code.astype(np.uint8) | sign
    code = np.where(nan, 0x7F | sign, code)
    return code.astype(np.uint8)


def f32_to_bf16_bits(x):
    """float32 -> bf16 bit pattern (uint16), round to nearest even."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def bf16_round(x):
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
