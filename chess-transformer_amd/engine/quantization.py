"""The int8 weights of a checkpoint: the module API of the reference's engine/quantization.py.

Produces {layer: {"projection" | "gate_up" | "down": (int8 N x K, f32 scale[N])}} for every block but the
last FP16_LAST_LAYERS, laid out as Int8Block reads them (reference quantization.py:122-140): projection
is Q | K | V | template_mix, gate_up the gate's rows then up's, down zero-padded to down_inputs(hidden)
and rotated by the block-diagonal Hadamard matrix / 32, so that (x H)(W H / 32)^T = x W^T. Rounding is
GPTQ (Frantar et al. 2022) in float64 on the input Hessians of calibration positions. The cache of
computed weights and its file names are the reference's (quantization.py:174-223), so a cached file
is found by either.

The calibration positions come from engine/Carlsen.pgn through python-chess, as in the reference;
where python-chess is not installed, callers pass encoded boards themselves.
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys
from contextlib import suppress
from pathlib import Path

import torch
from torch import nn

from model.checkpoint import load_model
from model.fused_blocks import link_input_mixes
from model.int8_blocks import DOWN_INPUT_MULTIPLE, HADAMARD_BLOCK, Int8Block, down_inputs, hadamard
from model.model import ChessTransformer

Int8Weights = dict[int, dict[str, tuple[torch.Tensor, torch.Tensor]]]

CARLSEN_PGN = Path(__file__).resolve().parent / "Carlsen.pgn"
CACHE_VARIABLE = "CHESS_TRANSFORMER_INT8_CACHE"


def cache_folder() -> Path | None:
    """The environment's named folder, else ~/.cache/chess_transformer/int8; None without a home folder."""
    if os.environ.get(CACHE_VARIABLE):
        return Path(os.environ[CACHE_VARIABLE])
    try:
        return Path.home() / ".cache" / "chess_transformer" / "int8"
    except RuntimeError:
        return None


CACHE = cache_folder()
# these name the cached file (with the rounding code's VERSION): the reference's production values
VERSION = 1
CALIBRATION_POSITIONS = 1024
CALIBRATION_FIRST_GAME = 1000
CALIBRATION_STEP = 9
DAMPENING = 0.01
GPTQ_COLUMNS = 128
FP16_LAST_LAYERS = 1
INT8_MAX = 127
CHOICE_VERSION = 1
ERROR_BATCH = 256


def calibration_positions():
    """Every CALIBRATION_STEP-th position of the Carlsen games after the first CALIBRATION_FIRST_GAME (reference :53-68)."""
    try:
        import chess.pgn
    except ImportError as error:
        raise ImportError("the calibration positions are read with python-chess; pass encoded boards instead") from error
    boards = []
    with open(CARLSEN_PGN) as pgn:
        for _ in range(CALIBRATION_FIRST_GAME):
            chess.pgn.skip_game(pgn)
        while len(boards) < CALIBRATION_POSITIONS and (game := chess.pgn.read_game(pgn)) is not None:
            board = game.board()
            for ply, move in enumerate(game.mainline_moves()):
                board.push(move)
                if board.is_game_over() or len(boards) == CALIBRATION_POSITIONS:
                    break
                if ply % CALIBRATION_STEP == CALIBRATION_STEP // 2:
                    boards.append(board.copy(stack=False))
    if len(boards) < CALIBRATION_POSITIONS:
        raise ValueError(f"{CARLSEN_PGN} has {len(boards)} calibration positions past game {CALIBRATION_FIRST_GAME}, not {CALIBRATION_POSITIONS}")
    return boards


def gptq(weight: torch.Tensor, hessian: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(int8 weight, f32 scale a row) of an N x K weight: columns rounded in order, each one's rounding error carried
    onto the columns not yet rounded through the inverse Hessian's upper Cholesky factor (GPTQ). float64 throughout,
    so that machines summing in other orders round every weight alike."""
    weight, hessian = weight.double().clone(), hessian.double().clone()
    columns = weight.shape[1]
    curvature = hessian.diagonal()
    # inputs that are always zero (down's padding) have no curvature: their weights stay zero
    never = curvature == 0
    curvature[never] = 1
    weight[:, never] = 0
    curvature += DAMPENING * curvature.mean()
    factor = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(hessian)), upper=True)
    scale = weight.abs().amax(dim=1).clamp(min=1e-20) / INT8_MAX
    integers = torch.zeros_like(weight)
    for first in range(0, columns, GPTQ_COLUMNS):
        last = min(first + GPTQ_COLUMNS, columns)
        part, part_factor = weight[:, first:last].clone(), factor[first:last, first:last]
        carried = torch.zeros_like(part)
        for i in range(last - first):
            rounded = (part[:, i] / scale).round().clamp(-INT8_MAX, INT8_MAX)
            integers[:, first + i] = rounded
            carried[:, i] = (part[:, i] - rounded * scale) / part_factor[i, i]
            part[:, i:] -= carried[:, i, None] * part_factor[i, i:]
        weight[:, last:] -= carried @ factor[first:last, last:]
    return integers.to(torch.int8), scale.float()


def nearest(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Round to nearest with a scale a row: gptq's answer for a diagonal Hessian, without its column loop."""
    weight = weight.double()
    scale = weight.abs().amax(dim=1).clamp(min=1e-20) / INT8_MAX
    return (weight / scale[:, None]).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8), scale.float()


@torch.no_grad()
def input_hessians(model: ChessTransformer, boards: torch.Tensor, batch: int = 128) -> list[dict[str, torch.Tensor]]:
    """Per block, the sum over the boards of x^T x of the inputs x of its projection, gate_up and down matmuls."""
    hessians: list[dict[str, torch.Tensor]] = [{} for _ in model.encoder]
    hooks = []
    for block, sums in zip(model.encoder, hessians):
        for name, layer in (("projection", block.Q), ("gate_up", block.mlp.gate_projection), ("down", block.mlp.down_projection)):
            def add(module, inputs, name=name, sums=sums):
                x = inputs[0].reshape(-1, inputs[0].shape[-1])
                sums[name] = sums.get(name, 0) + x.t() @ x
            hooks.append(layer.register_forward_pre_hook(add))
    try:
        for start in range(0, len(boards), batch):
            model(boards[start:start + batch].to(model.position_embed.device))
    finally:
        for hook in hooks:
            hook.remove()
    return hessians


def block_matrices(block) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """A block's projection and gate_up weights, its down weight padded and rotated, and that rotation."""
    projection = torch.cat([matmul.weight for matmul in (block.Q, block.K, block.V, block.template_mix)])
    gate_up = torch.cat([block.mlp.gate_projection.weight, block.mlp.up_projection.weight])
    hidden = block.mlp.down_projection.weight.shape[1]
    width = down_inputs(hidden)
    rotation = torch.block_diag(*[hadamard(HADAMARD_BLOCK)] * (width // HADAMARD_BLOCK)).to(block.mlp.down_projection.weight)
    down = nn.functional.pad(block.mlp.down_projection.weight, (0, width - hidden)) @ rotation / HADAMARD_BLOCK
    return projection, gate_up, down, rotation


@torch.no_grad()
def compute_int8_weights(model: ChessTransformer, boards: torch.Tensor) -> Int8Weights:
    """All but the last FP16_LAST_LAYERS blocks, GPTQ-rounded on the Hessians of boards (reference :124-140)."""
    hessians = input_hessians(model, boards)
    weights = {}
    for layer in range(len(hessians) - FP16_LAST_LAYERS):
        block, sums = model.encoder[layer], hessians[layer]
        projection, gate_up, down, rotation = block_matrices(block)
        padding = rotation.shape[0] - sums["down"].shape[0]
        padded = nn.functional.pad(sums["down"], (0, padding, 0, padding))
        weights[layer] = {"projection": gptq(projection, sums["projection"]), "gate_up": gptq(gate_up, sums["gate_up"]),
                          "down": gptq(down, rotation.t() @ padded @ rotation)}
    return weights


@torch.no_grad()
def nearest_int8_weights(model: ChessTransformer) -> Int8Weights:
    """compute_int8_weights with diagonal Hessians -- round to nearest, same layout -- for random-init networks that have no
    calibration positions worth the name (the benchmarks' networks)."""
    weights = {}
    for layer in range(len(model.encoder) - FP16_LAST_LAYERS):
        projection, gate_up, down, _ = block_matrices(model.encoder[layer])
        weights[layer] = {"projection": nearest(projection), "gate_up": nearest(gate_up), "down": nearest(down)}
    return weights


@torch.no_grad()
def block_errors(checkpoint_path: Path, weights: Int8Weights, boards: torch.Tensor | None = None, legal: torch.Tensor | None = None) -> dict[int, float]:
    """Per layer of weights, the policy's total variation over the legal moves between the fp16 model and the fp16 model with only
    that block in int8, mean over the calibration boards (reference :145-170). Without python-chess, pass boards and their
    legal-move masks (B x 1968 bool) -- or boards alone to take every move as legal."""
    from engine.inference import FP16_RESIDUAL_SCALE, answer_rows, fp16_model
    if boards is None:
        boards, legal = encoded_calibration()
    device = torch.device("cuda")
    boards = boards.to(device)
    legal = torch.ones(len(boards), answer_rows_width(checkpoint_path) - 1, dtype=torch.bool, device=device) if legal is None else legal.to(device)
    model = fp16_model(checkpoint_path)
    fp16_blocks = list(model.encoder)

    def priors(int8_blocks: dict[int, nn.Module]) -> torch.Tensor:
        blocks = [int8_blocks.get(layer, block) for layer, block in enumerate(fp16_blocks)]
        link_input_mixes(blocks)
        model.encoder = nn.ModuleList(blocks)
        logits = torch.cat([answer_rows(model(boards[start:start + ERROR_BATCH]))[:, :-1] for start in range(0, len(boards), ERROR_BATCH)])
        return torch.softmax(logits.double().masked_fill(~legal, -torch.inf), dim=-1)

    fp16_priors = priors({})
    errors = {}
    for layer, matmuls in weights.items():
        int8_priors = priors({layer: Int8Block(fp16_blocks[layer], matmuls, FP16_RESIDUAL_SCALE)})
        errors[layer] = 0.5 * (int8_priors - fp16_priors).abs().sum(dim=-1).mean().item()
    del model
    torch.cuda.empty_cache()
    return errors


def answer_rows_width(checkpoint_path: Path) -> int:
    from model.encoding import NUM_MOVE_IDS
    return NUM_MOVE_IDS + 1


def encoded_calibration() -> tuple[torch.Tensor, torch.Tensor]:
    """The calibration positions encoded, with their legal-move masks (python-chess)."""
    positions = calibration_positions()
    from model.encoding import NUM_MOVE_IDS, move_id
    import chess
    tokens, legal = [], torch.zeros(len(positions), NUM_MOVE_IDS, dtype=torch.bool)
    for row, board in enumerate(positions):
        tokens.append(encode_board(board))
        promotion = lambda move: move.promotion
        legal[row, [move_id(move.from_square, move.to_square, promotion(move), board.turn == chess.WHITE) for move in board.legal_moves]] = True
    return torch.tensor(tokens, dtype=torch.long), legal


def encode_board(board) -> list[int]:
    """A python-chess board as its 70 tokens, seen from the side to move (reference model/encoding.py:72-92)."""
    import chess
    from model.encoding import CASTLING_TOKEN_OFFSET, EN_PASSANT_TOKEN_OFFSET, NUM_PIECE_TYPES, TURN_TOKEN_OFFSET
    turn, opponent = board.turn, not board.turn
    flip = 0 if turn == chess.WHITE else 56
    tokens = [0] * 64
    for piece_type in chess.PIECE_TYPES:
        for square in chess.scan_forward(board.pieces_mask(piece_type, turn)):
            tokens[square ^ flip] = piece_type
        for square in chess.scan_forward(board.pieces_mask(piece_type, opponent)):
            tokens[square ^ flip] = piece_type + NUM_PIECE_TYPES
    en_passant = board.ep_square ^ flip if board.ep_square is not None and board.has_legal_en_passant() else 0
    return tokens + [TURN_TOKEN_OFFSET + (1 if turn == chess.WHITE else 0),
                     CASTLING_TOKEN_OFFSET + int(board.has_kingside_castling_rights(turn)),
                     CASTLING_TOKEN_OFFSET + int(board.has_queenside_castling_rights(turn)),
                     CASTLING_TOKEN_OFFSET + int(board.has_kingside_castling_rights(opponent)),
                     CASTLING_TOKEN_OFFSET + int(board.has_queenside_castling_rights(opponent)),
                     EN_PASSANT_TOKEN_OFFSET + en_passant]


def cached_weights_path(checkpoint_path: Path, fp16_blocks: int) -> Path | None:
    """CACHE / "<sha256 of the checkpoint>_<sha256 of the rounding settings, 16 hex>.pt"; a count of 0 stays out of the name."""
    if CACHE is None:
        return None
    with open(checkpoint_path, "rb") as checkpoint:
        digest = hashlib.file_digest(checkpoint, "sha256").hexdigest() if hasattr(hashlib, "file_digest") else hashlib.sha256(checkpoint.read()).hexdigest()
    rounding = (VERSION, CALIBRATION_POSITIONS, CALIBRATION_FIRST_GAME, CALIBRATION_STEP, DAMPENING, GPTQ_COLUMNS, FP16_LAST_LAYERS,
                HADAMARD_BLOCK, DOWN_INPUT_MULTIPLE)
    if fp16_blocks:
        rounding += (CHOICE_VERSION, fp16_blocks)
    return CACHE / f"{digest}_{hashlib.sha256(repr(rounding).encode()).hexdigest()[:16]}.pt"


def int8_weights(checkpoint_path: Path, fp16_blocks: int, boards: torch.Tensor | None = None, legal: torch.Tensor | None = None) -> Int8Weights:
    """The checkpoint's int8 weights on the cpu, from CACHE or computed on the gpu and cached, without the fp16_blocks blocks of the
    largest block_errors (reference :188-207). boards (and legal) replace the calibration positions where python-chess is absent."""
    if fp16_blocks < 0:
        raise ValueError(f"a count of blocks to keep in fp16, not {fp16_blocks}")
    path = cached_weights_path(checkpoint_path, fp16_blocks)
    if path is not None and path.exists():
        return torch.load(path, weights_only=True)
    if fp16_blocks:
        weights = int8_weights(checkpoint_path, 0, boards, legal)
        errors = block_errors(checkpoint_path, weights, boards, legal)
        kept = sorted(errors, key=errors.get, reverse=True)[:fp16_blocks]
        weights = {layer: matmuls for layer, matmuls in weights.items() if layer not in kept}
    else:
        if boards is None:
            boards, _ = encoded_calibration()
        #fp64 but the heads, whose inputs the model casts to fp32
        model = load_model(checkpoint_path, torch.device("cuda")).half_except_heads(torch.float64)
        weights = {layer: {name: tuple(tensor.cpu() for tensor in pair) for name, pair in matmuls.items()}
                   for layer, matmuls in compute_int8_weights(model, boards).items()}
        del model
        torch.cuda.empty_cache()
    cache_weights(weights, path)
    return weights


def cache_weights(weights: Int8Weights, path: Path | None) -> None:
    """Written under another name first, then moved: engines starting together compute the same weights."""
    if path is None:
        print("the int8 weights are not cached: there is no home folder", file=sys.stderr)
        return
    partial = path.with_name(f"{path.name}.{os.getpid()}.partial")
    try:
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save(weights, partial)
        os.replace(partial, path)
    except (OSError, RuntimeError) as error:
        with suppress(OSError):
            partial.unlink()
        print(f"the int8 weights are not cached: {error}", file=sys.stderr)


if __name__ == "__main__":
    parser = argparse.ArgumentParser(description="the int8 weights of a checkpoint, computed and cached")
    parser.add_argument("checkpoint", type=Path)
    parser.add_argument("--fp16-blocks", type=int, default=1, help="blocks kept in fp16 besides the last (the engine's ENGINE_FP16_BLOCKS)")
    parser.add_argument("--path", action="store_true", help="print the cached file's path and stop: nothing is computed, and no gpu is needed")
    arguments = parser.parse_args()
    path = cached_weights_path(arguments.checkpoint, arguments.fp16_blocks)
    if arguments.path:
        if path is None:
            raise SystemExit("the int8 weights have no cached file: there is no home folder")
        print(path)
        raise SystemExit
    weights = int8_weights(arguments.checkpoint, arguments.fp16_blocks)
    if path is None or not path.exists():
        raise SystemExit("the int8 weights could not be cached, which is what this is for: the engine would compute them at its first isready")
    print(path)
