"""Writes tests/golden/positions.npz: 4,096 seeded random legal positions as the network's tokens (uint8 [4096, 70]) and the
plies each took, for the benchmark's configs 0, 3 and 4 (positions reached by 0-80 uniformly random legal moves from the start
position). The reference draws them with python-chess, which is not installed here; tests/golden/chess_rules.py is this
repository's own move generator, pinned by perft and by the reference's encoding known answers.

    python tests/golden/make_positions.py            # about two minutes on one core
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from chess_rules import random_position  # noqa: E402

COUNT, SEED, MOST_PLIES = 4096, 20260, 80
OUT = HERE / "positions.npz"


def main() -> None:
    rng = np.random.default_rng(SEED)
    tokens = np.zeros((COUNT, 70), dtype=np.uint8)
    plies = np.zeros(COUNT, dtype=np.int16)
    for index in range(COUNT):
        position, plies[index] = random_position(rng, MOST_PLIES)
        tokens[index] = position.tokens()
    np.savez_compressed(OUT, tokens=tokens, plies=plies, seed=np.int64(SEED), most_plies=np.int64(MOST_PLIES))
    print(f"{OUT}: {COUNT} positions, plies {plies.min()}..{plies.max()} (mean {plies.mean():.1f})")


if __name__ == "__main__":
    main()
