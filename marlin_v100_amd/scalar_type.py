"""Weight element types of the Marlin ops and their integer ids.

The id is part of the op ABI: marlin_gemm / moe_wna16_marlin_gemm take `b_q_type.id`, so the
id of every type here equals vllm's (reference vllm/scalar_type.py:25-43; values pinned by
tests/golden/scalar_type_ids.json).  An id packs the type's fields least significant first:

    exponent:8 | mantissa:8 | signed:1 | bias:32 | finite_values_only:1 | nan_repr:8

`ScalarType.from_id` decodes those bits, so every id round-trips to the type that made it.
The public names (`ScalarType`, `NanRepr`, `scalar_types.*`, `.id`, `.size_bits`,
`from_id`) are the ones callers of the reference use.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum


class NanRepr(Enum):
    NONE = 0                # no NaN encoding
    IEEE_754 = 1            # NaN = all-ones exponent with a non-zero mantissa
    EXTD_RANGE_MAX_MIN = 2  # NaN = the all-ones pattern (extended range, e.g. e4m3fn)


# (attribute, bit width) in id order, least significant first
_LAYOUT = (("exponent", 8), ("mantissa", 8), ("signed", 1), ("bias", 32),
           ("_finite_values_only", 1), ("nan_repr", 8))
_ID_BITS = sum(w for _, w in _LAYOUT)


def _field_value(t: "ScalarType", attr: str) -> int:
    v = getattr(t, attr)
    return v.value if isinstance(v, NanRepr) else int(v)


@dataclass(frozen=True)
class ScalarType:
    exponent: int
    mantissa: int
    signed: bool
    bias: int = 0
    _finite_values_only: bool = False
    nan_repr: NanRepr = NanRepr.IEEE_754
    _id: int = field(default=0, init=False, repr=False, compare=False)

    def __post_init__(self):
        packed, shift = 0, 0
        for attr, width in _LAYOUT:
            packed |= (_field_value(self, attr) & ((1 << width) - 1)) << shift
            shift += width
        object.__setattr__(self, "_id", packed)

    @property
    def id(self) -> int:
        return self._id

    @property
    def size_bits(self) -> int:
        return self.exponent + self.mantissa + int(self.signed)

    def is_floating_point(self) -> bool:
        return self.exponent != 0

    def is_integer(self) -> bool:
        return self.exponent == 0

    def has_bias(self) -> bool:
        return self.bias != 0

    @classmethod
    def from_id(cls, scalar_type_id: int) -> "ScalarType":
        if not 0 <= scalar_type_id < (1 << _ID_BITS):
            raise ValueError(f"scalar_type_id {scalar_type_id} doesn't exist.")
        vals, rest = {}, scalar_type_id
        for attr, width in _LAYOUT:
            vals[attr], rest = rest & ((1 << width) - 1), rest >> width
        try:
            nan = NanRepr(vals["nan_repr"])
        except ValueError:
            raise ValueError(f"scalar_type_id {scalar_type_id} doesn't exist.") from None
        return cls(vals["exponent"], vals["mantissa"], bool(vals["signed"]), vals["bias"],
                   bool(vals["_finite_values_only"]), nan)

    @classmethod
    def uint(cls, size_bits: int, bias: int | None = None) -> "ScalarType":
        return cls(0, size_bits, False, bias or 0)

    @classmethod
    def int_(cls, size_bits: int, bias: int | None = None) -> "ScalarType":
        return cls(0, size_bits - 1, True, bias or 0)

    @classmethod
    def float_(cls, exponent: int, mantissa: int, finite_values_only: bool,
               nan_repr: NanRepr) -> "ScalarType":
        return cls(exponent, mantissa, True, 0, finite_values_only, nan_repr)

    @classmethod
    def float_IEEE754(cls, exponent: int, mantissa: int) -> "ScalarType":
        return cls(exponent, mantissa, True, 0, False, NanRepr.IEEE_754)

    def __str__(self) -> str:
        name = _NAMES.get(self.id)
        if name is not None:
            return name
        kind = "float" if self.is_floating_point() else ("int" if self.signed else "uint")
        return f"{kind}(e{self.exponent}m{self.mantissa}, bias={self.bias})"


class scalar_types:
    """The weight types the Marlin ops take (and the MXFP4 scale type)."""
    uint4 = ScalarType.uint(4)
    uint4b8 = ScalarType.uint(4, 8)
    uint8 = ScalarType.uint(8)
    uint8b128 = ScalarType.uint(8, 128)
    float4_e2m1f = ScalarType.float_(2, 1, True, NanRepr.NONE)
    float8_e4m3fn = ScalarType.float_(4, 3, True, NanRepr.EXTD_RANGE_MAX_MIN)
    float8_e8m0fnu = ScalarType(8, 0, False, 0, True, NanRepr.EXTD_RANGE_MAX_MIN)
    float16_e5m10 = ScalarType.float_IEEE754(5, 10)
    float16_e8m7 = ScalarType.float_IEEE754(8, 7)


_NAMES = {t.id: n for n, t in vars(scalar_types).items() if isinstance(t, ScalarType)}
