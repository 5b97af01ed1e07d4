"""Enums mirrored from the reference's kernel library call signatures
(attention_decode.py:1275, :1309; qkv.py:672-730).  The reference imports
them from nkilib.core.utils.common_types and only compares members by
identity, so the member names are the contract; the values are this
package's own."""
import enum


class QuantizationType(enum.Enum):
    NONE = 0
    STATIC = 1
    ROW = 2


class NormType(enum.Enum):
    NO_NORM = 0
    RMS_NORM = 1
    LAYER_NORM = 2
    RMS_NORM_SKIP_GAMMA = 3


class QKVOutputLayout(enum.Enum):
    BSD = 0
    NBSd = 1
    NBdS = 2


class QKVWeightLayout(enum.Enum):
    CONTIGUOUS = 0
