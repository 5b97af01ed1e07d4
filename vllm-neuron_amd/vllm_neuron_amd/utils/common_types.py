"""Enum mirrored from the reference's kernel library call signature
(attention_decode.py:1275, :1309)."""
import enum


class QuantizationType(enum.Enum):
    NONE = 0
    STATIC = 1
