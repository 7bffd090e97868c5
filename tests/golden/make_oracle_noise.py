"""Writes tests/golden/network_d512x28_noise.npz: how far two correct CPU restatements of the benchmarked int8 network drift
apart on the 1,024 positions of network_d512x28.npz. The second restatement is the oracle with one change, its fp16
linear (the combine and the fp16 block's matmuls; the reference sums these in fp16, model/fused_blocks.py:291) summed in
float32 instead of float64. The int8 re-quantisation of every block turns such rounding differences into int8 flips
that travel to the logits, so this is the precision at which an argmax can be called at all: positions whose top two
logits are closer than it are ties for any implementation that is not bit-identical to the float64 oracle.

    python tests/golden/make_oracle_noise.py         # about 6 minutes on 8 cores
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

FIXTURE, OUT, CHUNK = HERE / "network_d512x28.npz", HERE / "network_d512x28_noise.npz", 16
_network = None


def f32_linear(x, weight, bias=None, residual=None, gated=False, accumulate_fp32=False, original=None, residual_scale=None, input_scale=None):
    """oracle.int8_ops.linear with the products summed in float32 (the epilogue in float64 as there)."""
    K, width = weight.shape
    N = width // 2 if gated else width
    sums = (np.asarray(x).reshape(-1, K).astype(np.float32) @ np.asarray(weight).astype(np.float32)).astype(np.float64)
    out = sums[:, :N]
    if bias is not None:
        out = out + np.asarray(bias).astype(np.float64)[None, :]
    if gated:
        out = out / (1.0 + np.exp(-out)) * sums[:, N:]
    if residual is not None:
        out = out + np.asarray(residual).reshape(-1, N).astype(np.float64)
    dtype = np.float32 if accumulate_fp32 else np.float16
    if original is not None:
        stream = out.astype(dtype).astype(np.float64)
        rs = float(np.asarray(residual_scale, dtype=np.float32).reshape(-1)[0])
        is_ = float(np.asarray(input_scale, dtype=np.float32).reshape(-1)[0])
        out = rs * stream + is_ * np.asarray(original).reshape(-1, N).astype(np.float64)
    return out.astype(dtype).reshape(*np.asarray(x).shape[:-1], N)


def _build():
    global _network
    import torch
    torch.set_num_threads(1)
    from bench import SETTINGS, synthetic_model
    from engine.quantization import nearest_int8_weights
    from oracle import int8_ops
    int8_ops.linear = f32_linear
    model = synthetic_model(SETTINGS, int(np.load(FIXTURE)["seed"]))
    _network = ({name: value.clone() for name, value in model.state_dict().items()}, nearest_int8_weights(model))


def _outputs(first: int):
    from bench import SETTINGS, legal_boards
    from oracle import network
    state, weights = _network
    logits, _ = network.int8_forward(state, SETTINGS, weights, legal_boards(CHUNK, first))
    return first, logits.numpy()


def main() -> None:
    start = time.time()
    expected = np.load(FIXTURE)["logits"]
    found = np.zeros_like(expected)
    with Pool(7, initializer=_build) as pool:
        for first, logits in pool.imap_unordered(_outputs, range(0, len(expected), CHUNK)):
            found[first:first + CHUNK] = logits
    difference = np.abs(found - expected)
    agreement = float((found.argmax(-1) == expected.argmax(-1)).mean())
    np.savez_compressed(OUT, max_logit_difference=np.float64(difference.max()), mean_logit_difference=np.float64(difference.mean()),
                        argmax_agreement=np.float64(agreement), argmax=found.argmax(-1).astype(np.int16))
    print(f"{OUT}: max logit difference {difference.max():.3e}, mean {difference.mean():.3e}, argmax agreement {agreement:.4f}, "
          f"{time.time() - start:.0f} s")


if __name__ == "__main__":
    main()
