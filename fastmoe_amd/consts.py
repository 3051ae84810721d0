"""Implementation selector of the MoE combine (mirrors src/fastmoe/consts.py:4-6).

The reference declares it as an ``enum.StrEnum`` (Python >= 3.11); this ``str``-mixin Enum
compares equal to the same strings on Python 3.10.
"""
from enum import Enum


class MoEImplementation(str, Enum):
    FAST = "fast"
    STANDARD = "standard"

    def __str__(self) -> str:
        return self.value
