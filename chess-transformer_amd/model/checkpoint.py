"""Checkpoints as the reference writes them: {"model_settings": ..., "state_dict": ...} (reference model/checkpoint.py:22-42)."""
from __future__ import annotations

from pathlib import Path

import torch

from model.model import ChessTransformer


def save_checkpoint(model: ChessTransformer, model_settings: dict, checkpoint_path: Path) -> None:
    torch.save({"model_settings": model_settings, "state_dict": model.state_dict()}, checkpoint_path)


def load_checkpoint(checkpoint_path: Path, device: torch.device) -> tuple[ChessTransformer, dict]:
    """The model in training mode and its settings; a checkpoint that runs its blocks more than once is refused."""
    checkpoint = torch.load(checkpoint_path, map_location=device, weights_only=True)
    model_settings = dict(checkpoint["model_settings"])
    if model_settings.pop("loops", 1) != 1:
        raise ValueError(f"{checkpoint_path} runs its blocks more than once (loops in its settings), which the model here cannot")
    model = ChessTransformer(**model_settings)
    model.load_state_dict(checkpoint["state_dict"])
    return model.to(device), model_settings


def load_model(checkpoint_path: Path, device: torch.device) -> ChessTransformer:
    model, _ = load_checkpoint(checkpoint_path, device)
    return model.eval()
