"""The random streams of the reference trainer, reproduced draw for draw.

The reference shuffles items and draws the objective's noise with .NET's ``System.Random(int seed)``
(Trainer.cs:117-118, 242-249; RlcdObjective.cs:37-51, 157-163). That class is part of the .NET base
class library (the reference targets net10.0, Directory.Build.props:14-15), not of the reference.
A seeded ``System.Random`` uses the legacy algorithm every .NET version has kept for seeded instances:
Knuth's subtractive generator (TAOCP vol. 2 §3.2.2; Numerical Recipes' ``ran3``), with .NET's seeding:
a 56-entry table of which entries 1..55 are used, filled at stride 21 from ``161803398 − |seed|``,
then stirred four times with lag 31, and read with the two cursors starting at 0 and 21.
``Sample()`` is the next value times 1/(2³¹ − 1); ``Next(n)`` truncates ``Sample()·n``.

Restating it lets a run of this trainer see the same item order and the same Gaussian draws as the
reference trainer with the same seed.
"""
from __future__ import annotations

import math
from typing import List, MutableSequence

INT_MAX = 2 ** 31 - 1
_SEED_BASE = 161803398


class DotNetRandom:
    """``System.Random(seed)`` of .NET (the seeded, subtractive-generator implementation)."""

    def __init__(self, seed: int):
        seed = int(seed)
        if not -2 ** 31 <= seed < 2 ** 31:
            raise ValueError("seed must be a 32-bit signed integer")
        table = [0] * 56
        mj = _SEED_BASE - (INT_MAX if seed == -2 ** 31 else abs(seed))
        table[55] = mj
        mk, ii = 1, 0
        for _ in range(1, 55):
            ii = (ii + 21) % 55
            table[ii] = mk
            mk = mj - mk
            if mk < 0:
                mk += INT_MAX
            mj = table[ii]
        for _ in range(4):
            for i in range(1, 56):
                table[i] -= table[1 + (i + 30) % 55]
                if table[i] < 0:
                    table[i] += INT_MAX
        self._table = table
        self._next = 0
        self._nextp = 21

    def _sample_int(self) -> int:
        a = self._next + 1 if self._next + 1 < 56 else 1
        b = self._nextp + 1 if self._nextp + 1 < 56 else 1
        v = self._table[a] - self._table[b]
        if v == INT_MAX:
            v -= 1
        if v < 0:
            v += INT_MAX
        self._table[a] = v
        self._next, self._nextp = a, b
        return v

    def next_double(self) -> float:
        """``NextDouble()``: a double in [0, 1)."""
        return self._sample_int() * (1.0 / INT_MAX)

    def next(self, max_value: int | None = None) -> int:
        """``Next()`` (a value in [0, 2³¹ − 1)) or ``Next(max_value)`` (in [0, max_value))."""
        if max_value is None:
            return self._sample_int()
        if max_value < 0:
            raise ValueError("max_value must be non-negative")
        return int(self.next_double() * max_value)

    def next_range(self, lo: int, hi: int) -> int:
        """``Next(lo, hi)`` for ranges below 2³¹ (every range this package draws)."""
        if lo > hi:
            raise ValueError("lo must not exceed hi")
        span = hi - lo
        if span > INT_MAX:
            raise ValueError("ranges of 2^31 or more are not drawn here")
        return int(self.next_double() * span) + lo

    def shuffle_span(self, values: MutableSequence) -> None:
        """``Random.Shuffle(Span<T>)``: for i = 0..n−2, swap i with Next(i, n)."""
        n = len(values)
        for i in range(n - 1):
            j = self.next_range(i, n)
            if j != i:
                values[i], values[j] = values[j], values[i]

    def state(self) -> dict:
        """The generator's whole state, for a checkpoint."""
        return {"table": list(self._table), "next": self._next, "nextp": self._nextp}

    @classmethod
    def from_state(cls, state: dict) -> "DotNetRandom":
        r = cls.__new__(cls)
        r._table = [int(v) for v in state["table"]]
        r._next, r._nextp = int(state["next"]), int(state["nextp"])
        if len(r._table) != 56:
            raise ValueError("a generator state has 56 table entries")
        return r


def trainer_shuffle(values: List, rng: DotNetRandom) -> None:
    """Trainer.Shuffle (Trainer.cs:242-249): Fisher–Yates from the end, j = Next(i + 1)."""
    for i in range(len(values) - 1, 0, -1):
        j = rng.next(i + 1)
        values[i], values[j] = values[j], values[i]


def gaussian(rng: DotNetRandom) -> float:
    """RlcdObjective.Gaussian (RlcdObjective.cs:157-163): Box–Muller on 1 − NextDouble() and NextDouble()."""
    u1 = 1.0 - rng.next_double()
    u2 = rng.next_double()
    return math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
