"""Writes tests/golden/network_d512x28.npz: the CPU oracle's outputs (oracle/network.py int8_forward) for the first 1,024
positions of tests/golden/positions.npz through the benchmarked network -- bench.py's synthetic d512 x 28 int8 network
(27 int8 blocks and the fp16 last, random-init weights from numpy's generator, round-to-nearest int8 weights) -- so that
the GPU test checks the north star's bars (logits within 2e-2, argmax equal on at least 99.9% of positions, value within
5e-3) on 1,024 positions without running the oracle on the GPU box.

    python tests/golden/make_network_outputs.py      # about 10 minutes on 8 cores
"""
from __future__ import annotations

import sys
import time
from multiprocessing import Pool
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for path in (ROOT, ROOT / "chess-transformer_amd"):
    sys.path.insert(0, str(path))

COUNT, CHUNK, SEED = 1024, 16, 0
OUT = HERE / "network_d512x28.npz"
_network = None


def _build():
    global _network
    import torch
    torch.set_num_threads(1)
    from bench import SETTINGS, synthetic_model
    from engine.quantization import nearest_int8_weights
    model = synthetic_model(SETTINGS, SEED)
    _network = ({name: value.clone() for name, value in model.state_dict().items()}, nearest_int8_weights(model))


def _outputs(first: int):
    from bench import SETTINGS, legal_boards
    from oracle import network
    state, weights = _network
    logits, values = network.int8_forward(state, SETTINGS, weights, legal_boards(CHUNK, first))
    return first, logits.numpy(), values.numpy()


def main() -> None:
    from bench import SETTINGS, legal_boards
    start = time.time()
    logits = np.zeros((COUNT, 1968), dtype=np.float32)
    values = np.zeros((COUNT, SETTINGS["value_bins"]), dtype=np.float32)
    with Pool(7, initializer=_build) as pool:
        for first, chunk_logits, chunk_values in pool.imap_unordered(_outputs, range(0, COUNT, CHUNK)):
            logits[first:first + CHUNK], values[first:first + CHUNK] = chunk_logits, chunk_values
            print(f"positions {first}..{first + CHUNK - 1} done at {time.time() - start:.0f} s", flush=True)
    boards = legal_boards(COUNT).numpy().astype(np.uint8)
    np.savez_compressed(OUT, boards=boards, logits=logits, value_logits=values, seed=np.int64(SEED))
    print(f"{OUT}: {COUNT} positions in {time.time() - start:.0f} s")


if __name__ == "__main__":
    main()
