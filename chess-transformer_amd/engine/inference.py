"""The networks the engine evaluates, built as the reference's engine/inference.py builds them (:19-23, 238-278):
answer_rows, FP16_RESIDUAL_SCALE, fp16_model and int8_model. The reference's own inference module (its CUDA-graph
lanes, serving loop and the native round loop's address table) calls model.int8_blocks and engine.quantization and
runs over this package unchanged; this module is what this package's tests and benchmark build their networks with.
"""
from __future__ import annotations

from pathlib import Path

import torch
from torch import nn

from model.checkpoint import load_model
from model.model import expected_score

#scales the residual stream down so its channels stay below fp16's largest number, 65,504
FP16_RESIDUAL_SCALE = 1 / 16


#a row per board: the move logits, then the expected score
def answer_rows(outputs: tuple[torch.Tensor, torch.Tensor] | torch.Tensor) -> torch.Tensor:
    if isinstance(outputs, torch.Tensor):
        return outputs
    move_logits, value_logits = outputs
    return torch.cat([move_logits.float(), expected_score(value_logits).unsqueeze(1)], dim=1)


def fused_model(model: nn.Module) -> nn.Module:
    """An fp32 ChessTransformer (on the GPU) as the fp16 inference network: residual stream scaled by 1/16, all but the heads in fp16."""
    from model.fused_blocks import FusedTransformer
    return FusedTransformer(model.scale_residual_stream(FP16_RESIDUAL_SCALE).half_except_heads(torch.float16))


def fp16_model(checkpoint_path: Path) -> nn.Module:
    """The network in fp16 (f32 sums), the heads in fp32."""
    return fused_model(load_model(checkpoint_path, torch.device("cuda")))


def int8_model(checkpoint_path: Path, fp16_blocks: int, weights: dict | None = None) -> nn.Module:
    """fp16_model with every block in int8 but the last and the fp16_blocks whose int8 costs the policy most.
    weights: the rounded weights (engine/quantization.py) if already read, else rounded once per checkpoint."""
    from model.int8_blocks import quantize_blocks
    from engine.quantization import int8_weights
    if weights is None:
        weights = int8_weights(checkpoint_path, fp16_blocks)
    return quantize_blocks(fp16_model(checkpoint_path), weights, FP16_RESIDUAL_SCALE)


def int8_network(model: nn.Module, weights: dict) -> nn.Module:
    """int8_model for a model already in memory (fp32, on the GPU): the benchmark's and the tests' random-init networks."""
    from model.int8_blocks import quantize_blocks
    return quantize_blocks(fused_model(model), weights, FP16_RESIDUAL_SCALE)
