"""Pressure levels and their thresholds, as the precision controller takes
them (reference: src/microinfer/monitor.py:70-107).

Only what the plan needs lives here: a level is the machine's state, set by
the free device memory (headroom) against two thresholds. The polling
monitor that produces the headroom is outside this path.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass

MIB = 1 << 20


class Level(str, enum.Enum):
    """A pressure level: the machine's state, never a page's."""

    GREEN = "GREEN"
    YELLOW = "YELLOW"
    RED = "RED"


GREEN, YELLOW, RED = Level.GREEN, Level.YELLOW, Level.RED


@dataclass(frozen=True)
class Thresholds:
    """Headroom below `red_below_bytes` is RED, below `yellow_below_bytes`
    YELLOW, else GREEN; a new level must hold `persist_polls` polls."""

    red_below_bytes: int
    yellow_below_bytes: int
    persist_polls: int

    def __post_init__(self):
        if not 0 <= self.red_below_bytes < self.yellow_below_bytes:
            raise ValueError(f"thresholds nest, 0 <= red < yellow; got red below "
                             f"{self.red_below_bytes}, yellow below {self.yellow_below_bytes}")
        if self.persist_polls < 1:
            raise ValueError(f"a level holds for at least one poll; got {self.persist_polls}")

    def classify(self, headroom_bytes: int) -> Level:
        if headroom_bytes < self.red_below_bytes:
            return RED
        return YELLOW if headroom_bytes < self.yellow_below_bytes else GREEN


#: The reference's thresholds (ADR-0013): RED below 512 MiB, YELLOW below 1 GiB.
DEFAULT = Thresholds(red_below_bytes=512 * MIB, yellow_below_bytes=1024 * MIB, persist_polls=3)
