"""The int8 weights of a checkpoint: the module API of the reference's engine/quantization.py (int8_weights,
compute_int8_weights, gptq, block_errors, cached_weights_path, cache_folder and the settings that name the cache).

The result is {layer: {"projection" | "gate_up" | "down": (int8 [N, K], f32 scale [N])}} for every block but the last
FP16_LAST_LAYERS, in the layout Int8Block reads (reference quantization.py:122-140): projection is Q | K | V |
template_mix, gate_up the gate's rows then up's, and down zero-padded to down_inputs(hidden) and rotated by the
block-diagonal Sylvester matrix / 32, so that (x H)(W H / 32)^T = x W^T. Rounding is GPTQ (Frantar et al., 2022) in
float64 on the Hessians of each matmul's inputs over calibration positions; with a diagonal Hessian it is round to
nearest (nearest, nearest_int8_weights), which the random-init networks of the tests and the benchmark take.

The cache's file name is kept as the reference forms it -- the checkpoint's sha256 and a 16-hex-digit hash of the rounding
settings -- so that a cached file is found by either. The calibration positions are read with python-chess, which only
that step needs; without it, callers pass encoded boards (and their legal moves) themselves.
"""
from __future__ import annotations

import argparse
import hashlib
import os
import sys
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
    """The folder the environment names, else ~/.cache/chess_transformer/int8; None when there is no home folder."""
    named = os.environ.get(CACHE_VARIABLE)
    if named:
        return Path(named)
    try:
        home = Path.home()
    except RuntimeError:
        return None
    return home / ".cache" / "chess_transformer" / "int8"


CACHE = cache_folder()
# The rounding settings. With VERSION (of the rounding code) and, for a choice of fp16 blocks, CHOICE_VERSION, they name
# the cached file, in this order; the values are the reference's production ones.
VERSION = 1
CALIBRATION_POSITIONS = 1024
CALIBRATION_FIRST_GAME = 1000
CALIBRATION_STEP = 9
DAMPENING = 0.01
GPTQ_COLUMNS = 128
FP16_LAST_LAYERS = 1
CHOICE_VERSION = 1
INT8_MAX = 127
ERROR_BATCH = 256


def _row_scales(weight: torch.Tensor) -> torch.Tensor:
    return weight.abs().amax(dim=1).clamp(min=1e-20) / INT8_MAX


def nearest(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(int8, f32 scale a row): each row rounded to nearest on the grid of its absmax / 127, in float64."""
    weight = weight.double()
    scale = _row_scales(weight)
    return torch.round(weight / scale[:, None]).clamp(-INT8_MAX, INT8_MAX).to(torch.int8), scale.float()


def gptq(weight: torch.Tensor, hessian: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(int8, f32 scale a row) of an N x K weight by GPTQ, in float64.

    The inputs are rounded one at a time, in order. With U the upper Cholesky factor of the dampened Hessian's inverse, the
    rounding error of input j, scaled as e_j = (w_j - q_j s) / U[j, j], moves every later input i by -e_j U[j, i], which
    is the least-squares correction on the calibration inputs. Within a block of GPTQ_COLUMNS inputs each input gathers its
    corrections from the block's earlier errors when its turn comes (E[:, :j] @ U[:j, j]); a finished block's errors move
    all later blocks at once. Inputs that are always zero (down's padding) have no curvature: their weights are zero and
    stay zero."""
    W = weight.double().clone()
    H = hessian.double().clone()
    columns = W.shape[1]
    curvature = H.diagonal()
    dead = curvature == 0
    curvature[dead] = 1.0
    W[:, dead] = 0.0
    curvature += DAMPENING * curvature.mean()
    U = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(H)), upper=True)
    scale = _row_scales(W)
    integers = torch.empty_like(W)
    for start in range(0, columns, GPTQ_COLUMNS):
        stop = min(start + GPTQ_COLUMNS, columns)
        block, factor = W[:, start:stop], U[start:stop, start:stop]
        errors = torch.zeros_like(block)
        for j in range(stop - start):
            corrected = block[:, j] - errors[:, :j] @ factor[:j, j]
            rounded = torch.round(corrected / scale).clamp(-INT8_MAX, INT8_MAX)
            integers[:, start + j] = rounded
            errors[:, j] = (corrected - rounded * scale) / factor[j, j]
        W[:, stop:] -= errors @ U[start:stop, stop:]
    return integers.to(torch.int8), scale.float()


class HessianRecorder:
    """While open, sums x^T x in float64 over the inputs x of each block's three int8 matmuls: the projection (Q's input,
    which K, V and template_mix share), gate_up (the gate's input, which up shares) and down."""

    MATMULS = {"projection": lambda block: block.Q, "gate_up": lambda block: block.mlp.gate_projection, "down": lambda block: block.mlp.down_projection}

    def __init__(self, model: ChessTransformer):
        self.model = model
        self.sums: list[dict[str, torch.Tensor]] = [{} for _ in model.encoder]
        self.hooks = []

    def __enter__(self) -> "HessianRecorder":
        for sums, block in zip(self.sums, self.model.encoder):
            for name, layer in self.MATMULS.items():
                self.hooks.append(layer(block).register_forward_pre_hook(self._adder(sums, name)))
        return self

    @staticmethod
    def _adder(sums: dict, name: str):
        def add(module, inputs):
            rows = inputs[0].reshape(-1, inputs[0].shape[-1]).double()
            product = rows.t() @ rows
            sums[name] = product if name not in sums else sums[name] + product
        return add

    def __exit__(self, *exception) -> None:
        for hook in self.hooks:
            hook.remove()
        self.hooks.clear()


@torch.no_grad()
def input_hessians(model: ChessTransformer, boards: torch.Tensor, batch: int = 128) -> list[dict[str, torch.Tensor]]:
    """Per block, {matmul: the sum over boards of x^T x of that matmul's inputs}."""
    device = model.position_embed.device
    with HessianRecorder(model) as recorder:
        for part in boards.split(batch):
            model(part.to(device))
    return recorder.sums


def block_matrices(block) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """A block's projection and gate_up weights as Int8Block reads them, its down weight padded to down_inputs(hidden) and
    rotated by the block-diagonal Hadamard matrix / 32, and that rotation."""
    down = block.mlp.down_projection.weight
    width = down_inputs(down.shape[1])
    rotation = torch.kron(torch.eye(width // HADAMARD_BLOCK), hadamard(HADAMARD_BLOCK)).to(down)
    projection = torch.cat([block.Q.weight, block.K.weight, block.V.weight, block.template_mix.weight])
    gate_up = torch.cat([block.mlp.gate_projection.weight, block.mlp.up_projection.weight])
    rotated = nn.functional.pad(down, (0, width - down.shape[1])) @ rotation / HADAMARD_BLOCK
    return projection, gate_up, rotated, rotation


def int8_layers(model: ChessTransformer) -> range:
    return range(len(model.encoder) - FP16_LAST_LAYERS)


@torch.no_grad()
def compute_int8_weights(model: ChessTransformer, boards: torch.Tensor) -> Int8Weights:
    """GPTQ on the calibration boards' Hessians, for all but the last FP16_LAST_LAYERS blocks (reference :124-140). down's
    Hessian is of its rotated inputs: R^T H R over the zero-padded hidden units."""
    hessians = input_hessians(model, boards)
    weights = {}
    for layer in int8_layers(model):
        projection, gate_up, down, rotation = block_matrices(model.encoder[layer])
        sums = hessians[layer]
        padding = rotation.shape[0] - sums["down"].shape[0]
        rotated = rotation.t() @ nn.functional.pad(sums["down"], (0, padding, 0, padding)) @ rotation
        weights[layer] = {"projection": gptq(projection, sums["projection"]), "gate_up": gptq(gate_up, sums["gate_up"]), "down": gptq(down, rotated)}
    return weights


@torch.no_grad()
def nearest_int8_weights(model: ChessTransformer) -> Int8Weights:
    """compute_int8_weights with diagonal Hessians -- round to nearest, the same layout -- for random-init networks, which
    have no calibration positions worth the name (the tests' and the benchmark's)."""
    weights = {}
    for layer in int8_layers(model):
        projection, gate_up, down, _ = block_matrices(model.encoder[layer])
        weights[layer] = {"projection": nearest(projection), "gate_up": nearest(gate_up), "down": nearest(down)}
    return weights


@torch.no_grad()
def block_errors(checkpoint_path: Path, weights: Int8Weights, boards: torch.Tensor | None = None, legal: torch.Tensor | None = None) -> dict[int, float]:
    """Per layer of weights: the total variation distance between the policy over the legal moves of the fp16 network and
    of the fp16 network with that one block in int8, mean over the calibration boards (reference :145-170). Without
    python-chess pass the boards and their legal-move masks (B x 1968), or the boards alone to count every move legal."""
    from engine.inference import FP16_RESIDUAL_SCALE, answer_rows, fp16_model
    if boards is None:
        boards, legal = encoded_calibration()
    device = torch.device("cuda")
    boards = boards.to(device)
    model = fp16_model(checkpoint_path)
    originals = list(model.encoder)

    def policy(replaced: dict[int, nn.Module]) -> torch.Tensor:
        blocks = [replaced.get(layer, block) for layer, block in enumerate(originals)]
        link_input_mixes(blocks)
        model.encoder = nn.ModuleList(blocks)
        logits = torch.cat([answer_rows(model(part))[:, :-1] for part in boards.split(ERROR_BATCH)]).double()
        if legal is not None:
            logits = logits.masked_fill(~legal.to(device), -torch.inf)
        return torch.softmax(logits, dim=-1)

    baseline = policy({})
    errors = {layer: 0.5 * (policy({layer: Int8Block(originals[layer], matmuls, FP16_RESIDUAL_SCALE)}) - baseline).abs().sum(-1).mean().item()
              for layer, matmuls in weights.items()}
    del model
    torch.cuda.empty_cache()
    return errors


def calibration_positions():
    """Every CALIBRATION_STEP-th position (from the middle of each step) of the Carlsen games from game CALIBRATION_FIRST_GAME
    on, until CALIBRATION_POSITIONS: python-chess boards (reference :53-68)."""
    try:
        import chess.pgn
    except ImportError as error:
        raise ImportError("the calibration positions are read with python-chess; pass encoded boards instead") from error
    positions = []
    with open(CARLSEN_PGN) as pgn:
        for _ in range(CALIBRATION_FIRST_GAME):
            chess.pgn.skip_game(pgn)
        while len(positions) < CALIBRATION_POSITIONS:
            game = chess.pgn.read_game(pgn)
            if game is None:
                break
            board = game.board()
            for ply, move in enumerate(game.mainline_moves()):
                board.push(move)
                if board.is_game_over() or len(positions) == CALIBRATION_POSITIONS:
                    break
                if ply % CALIBRATION_STEP == CALIBRATION_STEP // 2:
                    positions.append(board.copy(stack=False))
    if len(positions) < CALIBRATION_POSITIONS:
        raise ValueError(f"{CARLSEN_PGN} has {len(positions)} calibration positions past game {CALIBRATION_FIRST_GAME}, not {CALIBRATION_POSITIONS}")
    return positions


def board_tokens(board) -> list[int]:
    """A python-chess board as the network's 70 tokens, seen from the side to move (the layout of model/encoding.py)."""
    import chess
    from model.encoding import CASTLING_TOKEN_OFFSET, EN_PASSANT_TOKEN_OFFSET, NUM_PIECE_TYPES, TURN_TOKEN_OFFSET
    mover = board.turn
    mirror = 0 if mover == chess.WHITE else 56
    tokens = [0] * 64
    for square, piece in board.piece_map().items():
        tokens[square ^ mirror] = piece.piece_type + (0 if piece.color == mover else NUM_PIECE_TYPES)
    rights = [board.has_kingside_castling_rights(mover), board.has_queenside_castling_rights(mover),
              board.has_kingside_castling_rights(not mover), board.has_queenside_castling_rights(not mover)]
    passing = board.ep_square ^ mirror if board.ep_square is not None and board.has_legal_en_passant() else 0
    return tokens + [TURN_TOKEN_OFFSET + int(mover == chess.WHITE)] + [CASTLING_TOKEN_OFFSET + int(right) for right in rights] \
        + [EN_PASSANT_TOKEN_OFFSET + passing]


def encoded_calibration() -> tuple[torch.Tensor, torch.Tensor]:
    """The calibration positions' tokens and legal-move masks (python-chess)."""
    import chess
    from model.encoding import NUM_MOVE_IDS, move_id
    positions = calibration_positions()
    legal = torch.zeros(len(positions), NUM_MOVE_IDS, dtype=torch.bool)
    for row, board in enumerate(positions):
        for move in board.legal_moves:
            legal[row, move_id(move.from_square, move.to_square, move.promotion, board.turn == chess.WHITE)] = True
    return torch.tensor([board_tokens(board) for board in positions], dtype=torch.long), legal


def rounding_settings(fp16_blocks: int) -> tuple:
    settings = (VERSION, CALIBRATION_POSITIONS, CALIBRATION_FIRST_GAME, CALIBRATION_STEP, DAMPENING, GPTQ_COLUMNS, FP16_LAST_LAYERS,
                HADAMARD_BLOCK, DOWN_INPUT_MULTIPLE)
    return settings + (CHOICE_VERSION, fp16_blocks) if fp16_blocks else settings


def cached_weights_path(checkpoint_path: Path, fp16_blocks: int) -> Path | None:
    """CACHE / "<checkpoint sha256>_<16 hex digits of the rounding settings' sha256>.pt"; a count of 0 stays out of the
    settings, so that files cached before the count existed are read. None without a cache folder."""
    if CACHE is None:
        return None
    content = hashlib.sha256()
    with open(checkpoint_path, "rb") as checkpoint:
        for chunk in iter(lambda: checkpoint.read(1 << 20), b""):
            content.update(chunk)
    settings = hashlib.sha256(repr(rounding_settings(fp16_blocks)).encode()).hexdigest()[:16]
    return CACHE / f"{content.hexdigest()}_{settings}.pt"


def int8_weights(checkpoint_path: Path, fp16_blocks: int, boards: torch.Tensor | None = None, legal: torch.Tensor | None = None) -> Int8Weights:
    """The checkpoint's int8 weights on the CPU: read from CACHE, or computed on the GPU and cached. fp16_blocks: the blocks
    of the largest block_errors kept out (reference :188-207). boards (and legal) stand in for the calibration positions
    where python-chess is absent."""
    if fp16_blocks < 0:
        raise ValueError(f"a count of blocks to keep in fp16, not {fp16_blocks}")
    path = cached_weights_path(checkpoint_path, fp16_blocks)
    if path is not None and path.exists():
        return torch.load(path, weights_only=True)
    if fp16_blocks:
        every = int8_weights(checkpoint_path, 0, boards, legal)
        errors = block_errors(checkpoint_path, every, boards, legal)
        worst = set(sorted(errors, key=errors.get, reverse=True)[:fp16_blocks])
        weights = {layer: matmuls for layer, matmuls in every.items() if layer not in worst}
    else:
        if boards is None:
            boards, _ = encoded_calibration()
        # float64 throughout but the heads, whose inputs the model casts to f32
        model = load_model(checkpoint_path, torch.device("cuda")).half_except_heads(torch.float64)
        computed = compute_int8_weights(model, boards)
        weights = {layer: {name: (integers.cpu(), scale.cpu()) for name, (integers, scale) in matmuls.items()} for layer, matmuls in computed.items()}
        del model
        torch.cuda.empty_cache()
    cache_weights(weights, path)
    return weights


def cache_weights(weights: Int8Weights, path: Path | None) -> None:
    """Saves weights at path by way of a file of this process's own, renamed into place, so that engines starting together
    never read half a file. A cache that cannot be written is reported and costs only the next start's time."""
    if path is None:
        print("the int8 weights are not cached: there is no cache folder (no home folder and no $" + CACHE_VARIABLE + ")", file=sys.stderr)
        return
    staging = path.parent / f".{path.name}.{os.getpid()}"
    try:
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save(weights, staging)
        os.replace(staging, path)
    except (OSError, RuntimeError) as error:
        try:
            staging.unlink()
        except OSError:
            pass
        print(f"the int8 weights are not cached at {path}: {error}", file=sys.stderr)


def main(arguments: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="compute a checkpoint's int8 weights and write them to the cache the engine reads")
    parser.add_argument("checkpoint", type=Path)
    parser.add_argument("--fp16-blocks", type=int, default=1, help="blocks besides the last to keep in fp16 (the engine's ENGINE_FP16_BLOCKS)")
    parser.add_argument("--path", action="store_true", help="only print where the cached file is or would be (no GPU needed)")
    options = parser.parse_args(arguments)
    path = cached_weights_path(options.checkpoint, options.fp16_blocks)
    if options.path or path is None:
        print(path if path is not None else f"no cache folder: set ${CACHE_VARIABLE}", file=sys.stdout if path else sys.stderr)
        return 0 if path is not None else 1
    weights = int8_weights(options.checkpoint, options.fp16_blocks)
    if not path.exists():
        print(f"computed, but {path} could not be written: the engine would compute the weights again at its start", file=sys.stderr)
        return 1
    print(path)
    print("int8 blocks:", sorted(weights))
    return 0


if __name__ == "__main__":
    sys.exit(main())
