"""The network's modules and weights: the reference's ChessTransformer (model/model.py), which FusedBlock / Int8Block are
built from and whose state_dict a checkpoint holds.

The module tree, parameter names and shapes are the reference's, so that a checkpoint ({"model_settings", "state_dict"},
reference model/checkpoint.py:22-23) loads here unchanged; that tree is the only part kept alike. The arithmetic is the
reference's network (model.py:71-99, 245-270) in a formulation of this build's own, used for the fp32/fp64 CPU forward
(calibration of the int8 weights, the CPU path) -- the GPU path runs the fused blocks instead:
  - a pre-RMSNorm block whose input is residual_scale * x + input_scale * embedding; grouped-query attention through
    scaled_dot_product_attention, the per-head q/k RMSNorms applied first and the template bias of the 64 squares passed
    as the additive mask (metadata rows and columns zero); a SwiGLU mlp;
  - 23 learned square-feature rows summed per square, found by run lengths along precomputed rays (how many empty
    squares precede the first piece) rather than by searching;
  - move logits from a from x to bilinear form, read at each move's (from, to) cell of the flattened 64 x 64 products,
    with the promotion logits added at the promotion moves; a 128-bin value head.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from model.encoding import (BOARD_VOCAB_SIZE, MOVE_FROM_SQUARES, MOVE_TO_SQUARES, NUM_PIECE_CODES, NUM_PIECE_TYPES, NUM_SQUARES,
                            PROMOTION_MOVE_IDS, PROMOTION_PIECES, PROMOTION_TO_SQUARES, TOKENS_PER_BOARD)

VALUE_TOKEN_DIM = 16          # board_down's width per token: the value head reads 70 x 16 numbers
VALUE_BINS = 128
MLP_WIDTH_MULTIPLE = 32
NORM_EPS = 1e-5
PROMOTION_PIECE_COUNT = 4     # knight, bishop, rook, queen


def mlp_hidden_width(d_model: int, mlp_ratio: float | None = None) -> int:
    """The SwiGLU width: ratio x d_model (8/3 unless given) rounded down to a multiple of 32, at least 32."""
    width = int((8 / 3 if mlp_ratio is None else mlp_ratio) * d_model)
    return max(MLP_WIDTH_MULTIPLE, width - width % MLP_WIDTH_MULTIPLE)


def value_bin_centres(bins: int, device: torch.device | None = None) -> torch.Tensor:
    """The midpoints of bins equal bins over [0, 1]."""
    return (torch.arange(bins, device=device, dtype=torch.float32) + 0.5) / bins


def expected_score(value_logits: torch.Tensor) -> torch.Tensor:
    """0 (lost) to 1 (won): the bin centres weighted by the value logits' softmax, in f32."""
    probabilities = torch.softmax(value_logits.float(), dim=-1)
    return (probabilities * value_bin_centres(value_logits.shape[-1], value_logits.device)).sum(-1)


class SwiGLU(nn.Module):
    def __init__(self, d_model: int, d_hidden: int):
        super().__init__()
        self.up_projection = nn.Linear(d_model, d_hidden, bias=False)
        self.gate_projection = nn.Linear(d_model, d_hidden, bias=False)
        self.down_projection = nn.Linear(d_hidden, d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate = self.gate_projection(x)
        return self.down_projection(gate * torch.sigmoid(gate) * self.up_projection(x))


class TransformerBlock(nn.Module):
    """One block. Attribute names are the state dict's; n_heads query heads of width d_qk_head (qk_ratio of d_head) share
    kv_heads key/value heads (value width d_head = d_model / n_heads)."""

    def __init__(self, d_model: int, n_heads: int, position_templates: int, mlp_hidden: int, qk_ratio: float, kv_heads: int | None):
        super().__init__()
        self.d_model, self.n_heads, self.position_templates = d_model, n_heads, position_templates
        self.d_head = d_model // n_heads
        self.d_qk_head = max(1, round(qk_ratio * self.d_head))
        self.kv_heads = kv_heads or n_heads
        if n_heads % self.kv_heads:
            raise ValueError(f"{n_heads} heads cannot be split into groups for {self.kv_heads} key/value heads")
        self.heads_per_kv = n_heads // self.kv_heads
        self.Q = nn.Linear(d_model, n_heads * self.d_qk_head)
        self.K = nn.Linear(d_model, self.kv_heads * self.d_qk_head)
        self.V = nn.Linear(d_model, self.kv_heads * self.d_head)
        self.q_norm, self.k_norm = nn.RMSNorm(self.d_qk_head, eps=NORM_EPS), nn.RMSNorm(self.d_qk_head, eps=NORM_EPS)
        self.ln1, self.ln2 = nn.RMSNorm(d_model, eps=NORM_EPS), nn.RMSNorm(d_model, eps=NORM_EPS)
        self.combine_heads = nn.Linear(d_model, d_model)
        self.mlp = SwiGLU(d_model, mlp_hidden)
        self.template_mix = nn.Linear(d_model, position_templates * n_heads)
        self.residual_scale = nn.Parameter(torch.ones(1))
        self.input_scale = nn.Parameter(torch.zeros(1))

    def template_bias(self, normed: torch.Tensor, templates: torch.Tensor) -> torch.Tensor:
        """[B, heads, T, T]: on query square i and key square j, sum_t c[i, head, t] * templates[t, i, j], with c the
        template_mix of square i's row; zero on the metadata tokens' rows and columns."""
        B, T, _ = normed.shape
        mix = self.template_mix(normed[:, :NUM_SQUARES]).view(B, NUM_SQUARES, self.n_heads, 1, self.position_templates)
        # per query square i, its [1 x templates] coefficients times templates[:, i, :] ([templates x 64])
        squares = torch.matmul(mix.transpose(1, 2), templates.to(normed.dtype).transpose(0, 1)).squeeze(-2)
        bias = normed.new_zeros(B, self.n_heads, T, T)
        bias[:, :, :NUM_SQUARES, :NUM_SQUARES] = squares
        return bias

    def forward(self, x: torch.Tensor, templates: torch.Tensor, original_board_embed: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        stream = x * self.residual_scale + original_board_embed * self.input_scale
        normed = self.ln1(stream)
        split = lambda rows, count, width: rows.view(B, T, count, width).transpose(1, 2)
        q = split(self.q_norm(self.Q(normed).view(B, T, self.n_heads, self.d_qk_head)), self.n_heads, self.d_qk_head)
        k = split(self.k_norm(self.K(normed).view(B, T, self.kv_heads, self.d_qk_head)), self.kv_heads, self.d_qk_head)
        v = split(self.V(normed), self.kv_heads, self.d_head)
        attended = F.scaled_dot_product_attention(q, k, v, attn_mask=self.template_bias(normed, templates), enable_gqa=self.heads_per_kv > 1)
        stream = stream + self.combine_heads(attended.transpose(1, 2).reshape(B, T, self.d_model))
        return stream + self.mlp(self.ln2(stream))


# piece codes on the squares: 0 empty, 1-6 the side to move's pawn, knight, bishop, rook, queen, king, 7-12 the other side's
PAWN, KNIGHT, QUEEN, KING = 1, 2, 5, 6
THEIRS = NUM_PIECE_TYPES          # added to a piece code for the other side's piece
EDGE = NUM_PIECE_CODES            # the code past every edge of the board
# (file step, rank step): rank +1 is towards the other side, every board being seen from the side to move
DIRECTIONS = [(0, 1), (0, -1), (1, 0), (-1, 0), (1, 1), (-1, 1), (1, -1), (-1, -1)]
KNIGHT_JUMPS = [(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)]
NO_PIECE = 15 * 15                # the offset row when there is no such piece
# each feature's rows: where the square is from a piece, 15 x 15 + none; a neighbour's code or the edge; none or the first
# piece along a line (12 codes x 7 distances); our and their attacking knights, 0 / 1 / 2+ each; none or the nearest pawn
# up or down the file, ours or theirs, 7 distances
OFFSET_ROWS, NEIGHBOUR_ROWS, LINE_ROWS, KNIGHT_ROWS, PAWN_ROWS = NO_PIECE + 1, NUM_PIECE_CODES + 1, 1 + 12 * 7, 3 * 3, 1 + 2 * 7
RAY_LENGTH = 7


def _square_tables() -> tuple[torch.Tensor, torch.Tensor]:
    """rays [64, 8, 7]: the squares out along each direction, nearest first; jumps [64, 8]: the knight jumps; NUM_SQUARES for
    a square past the edge."""
    files, ranks = torch.arange(NUM_SQUARES) % 8, torch.arange(NUM_SQUARES) // 8
    distance = torch.arange(1, RAY_LENGTH + 1)

    def land(file_steps: torch.Tensor, rank_steps: torch.Tensor) -> torch.Tensor:
        file, rank = files.view(-1, *[1] * file_steps.dim()) + file_steps, ranks.view(-1, *[1] * rank_steps.dim()) + rank_steps
        inside = (file >= 0) & (file < 8) & (rank >= 0) & (rank < 8)
        return torch.where(inside, rank * 8 + file, NUM_SQUARES)

    steps = torch.tensor(DIRECTIONS)
    rays = land(steps[:, 0, None] * distance, steps[:, 1, None] * distance)
    jumps = torch.tensor(KNIGHT_JUMPS)
    return rays, land(jumps[:, 0], jumps[:, 1])


def _leading(run: torch.Tensor) -> torch.Tensor:
    """Along the last axis: how many leading entries hold (the run length before the first that does not)."""
    return run.long().cumprod(-1).sum(-1)


class SquareFeatures(nn.Module):
    """23 learned rows summed per square (the reference's model.py:128-174): where the two kings and queens are from the square,
    its 8 neighbours, the first piece along each of the 8 lines and how far, the knights attacking it, and the nearest pawn up
    and down its file. rays, knight_jumps and row_offsets are also what the GPU's board embedding reads."""

    def __init__(self, d_model: int):
        super().__init__()
        rows = torch.tensor([OFFSET_ROWS] * 4 + [NEIGHBOUR_ROWS] * 8 + [LINE_ROWS] * 8 + [KNIGHT_ROWS] + [PAWN_ROWS] * 2)
        self.register_buffer("row_offsets", rows.cumsum(0) - rows, persistent=False)
        # zeros: a new model starts without the features and draws no random numbers
        self.table = nn.Parameter(torch.zeros(int(rows.sum()), d_model))
        rays, jumps = _square_tables()
        self.register_buffer("rays", rays, persistent=False)
        self.register_buffer("knight_jumps", jumps, persistent=False)

    def indices(self, board_state: torch.Tensor) -> torch.Tensor:
        """B x 64 x 23: each square's row within each feature's rows."""
        squares = board_state[:, :NUM_SQUARES].long()
        B = squares.shape[0]
        board = torch.cat([squares, squares.new_full((B, 1), EDGE)], 1)        # square 64 is past the edge
        place = torch.arange(NUM_SQUARES, device=squares.device)
        columns = []
        for code in (KING, KING + THEIRS, QUEEN, QUEEN + THEIRS):
            found = torch.where(squares == code, place, NUM_SQUARES).amin(1, keepdim=True)     # the first such square, or 64
            offset = (place // 8 - found // 8 + 7) * 15 + place % 8 - found % 8 + 7
            columns.append(torch.where(found < NUM_SQUARES, offset, NO_PIECE))
        along = board[:, self.rays]                                            # B x 64 x 8 x 7 codes, nearest first
        empties = _leading(along == 0)                                         # empty squares before a piece or the edge
        met = along.gather(-1, empties.clamp(max=RAY_LENGTH - 1).unsqueeze(-1)).squeeze(-1)
        lines = torch.where((empties < RAY_LENGTH) & (met != EDGE), 1 + (met - 1) * RAY_LENGTH + empties, 0)
        jumps = board[:, self.knight_jumps]
        knights = (jumps == KNIGHT).sum(-1).clamp(max=2) * 3 + (jumps == KNIGHT + THEIRS).sum(-1).clamp(max=2)
        file = along[:, :, :2]                                                 # up and down the file
        others = _leading((file != PAWN) & (file != PAWN + THEIRS))            # squares before the first pawn, past any piece
        pawn = file.gather(-1, others.clamp(max=RAY_LENGTH - 1).unsqueeze(-1)).squeeze(-1)
        pawns = torch.where(others < RAY_LENGTH, 1 + (pawn == PAWN + THEIRS).long() * RAY_LENGTH + others, 0)
        return torch.cat([torch.stack(columns, -1), along[..., 0], lines, knights.unsqueeze(-1), pawns], -1)

    def forward(self, board_state: torch.Tensor) -> torch.Tensor:
        return self.table[self.indices(board_state) + self.row_offsets].sum(-2)


class ChessTransformer(nn.Module):
    HEADS = ("from_projection", "to_projection", "promotion_projection", "board_down_project", "eval_head")

    def __init__(self, d_model: int = 128, num_layers: int = 4, n_heads: int = 4, position_templates: int = 8, mlp_hidden: int | None = None,
                 qk_ratio: float | list[float] = 1.0, kv_heads: int | None = None, value_bins: int = VALUE_BINS):
        super().__init__()
        if value_bins < 2:
            raise ValueError(f"value_bins is the eval head's bins over the expected score, at least 2, got {value_bins}")
        ratios = list(qk_ratio) if isinstance(qk_ratio, (list, tuple)) else [qk_ratio] * num_layers
        if len(ratios) != num_layers:
            raise ValueError(f"{len(ratios)} qk ratios for {num_layers} blocks, give one or one per block")
        hidden = mlp_hidden_width(d_model) if mlp_hidden is None else mlp_hidden
        self.d_model = d_model
        self.embed = nn.Embedding(BOARD_VOCAB_SIZE, d_model)
        self.position_embed = nn.Parameter(torch.randn(TOKENS_PER_BOARD, d_model))
        self.square_features = SquareFeatures(d_model)
        self.templates = nn.Parameter(torch.zeros(position_templates, NUM_SQUARES, NUM_SQUARES))
        self.encoder = nn.ModuleList(TransformerBlock(d_model, n_heads, position_templates, hidden, ratio, kv_heads) for ratio in ratios)
        self.board_down_project = nn.Sequential(nn.Linear(d_model, VALUE_TOKEN_DIM), nn.GELU())
        self.eval_head = nn.Sequential(nn.Linear(TOKENS_PER_BOARD * VALUE_TOKEN_DIM, d_model), nn.GELU(), nn.Linear(d_model, value_bins))
        for name, values in (("from_squares", MOVE_FROM_SQUARES), ("to_squares", MOVE_TO_SQUARES), ("promotion_move_ids", PROMOTION_MOVE_IDS),
                             ("promotion_to_squares", PROMOTION_TO_SQUARES), ("promotion_pieces", PROMOTION_PIECES)):
            self.register_buffer(name, torch.tensor(values, dtype=torch.long))
        self.from_projection = nn.Linear(d_model, d_model)
        self.to_projection = nn.Linear(d_model, d_model)
        self.promotion_projection = nn.Linear(d_model, PROMOTION_PIECE_COUNT)
        self.ln = nn.RMSNorm(d_model, eps=NORM_EPS)

    def half_except_heads(self, dtype: torch.dtype = torch.bfloat16) -> "ChessTransformer":
        """Every parameter but the heads' in dtype; the heads stay as they are and read their inputs in f32."""
        with torch.no_grad():
            for name, parameter in self.named_parameters():
                if not name.startswith(self.HEADS):
                    parameter.data = parameter.data.to(dtype)
        return self

    def scale_residual_stream(self, scale: float) -> "ChessTransformer":
        """Everything written into the residual stream times scale: the embeddings and each block's combine_heads and down.
        Every read of the stream is an RMSNorm, so no output changes but through the norms' eps."""
        writers = [self.embed.weight, self.position_embed, self.square_features.table]
        for block in self.encoder:
            writers += [block.combine_heads.weight, block.combine_heads.bias, block.mlp.down_projection.weight]
        with torch.no_grad():
            for weight in writers:
                weight.mul_(scale)
        return self

    def embedding(self, board_state: torch.Tensor) -> torch.Tensor:
        tokens = self.embed(board_state) + self.position_embed
        return torch.cat([tokens[:, :NUM_SQUARES] + self.square_features(board_state), tokens[:, NUM_SQUARES:]], 1)

    def heads(self, model_output: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(move logits [B, 1968], value logits [B, bins]) of the final norm's rows, in f32."""
        with torch.autocast(device_type=model_output.device.type, enabled=False):
            squares = model_output[:, :NUM_SQUARES].float()
            products = torch.matmul(self.from_projection(squares), self.to_projection(squares).transpose(1, 2)) / math.sqrt(self.d_model)
            logits = products.flatten(1).index_select(1, self.from_squares * NUM_SQUARES + self.to_squares)
            promotions = self.promotion_projection(squares).flatten(1)
            cells = self.promotion_to_squares * PROMOTION_PIECE_COUNT + self.promotion_pieces
            logits = logits.index_add(1, self.promotion_move_ids, promotions.index_select(1, cells))
            values = self.eval_head(self.board_down_project(model_output.float()).flatten(1))
        return logits, values

    def forward(self, board_state: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        embedded = x = self.embedding(board_state)
        for block in self.encoder:
            x = block(x, self.templates, embedded)
        return self.heads(self.ln(x))
