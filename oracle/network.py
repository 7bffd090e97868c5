"""CPU restatement of the whole network -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module. It works from a
state_dict (the reference's checkpoint format, model/checkpoint.py:22-23) and never imports the product.

  square_feature_rows  model/model.py:128-174 (SquareFeatures.indices), by walking the board square by square
  input_embedding      model/fused_blocks.py:370-393 (input_embedding_kernel): the features summed in f32 in slot order
  fp32_forward         model/model.py:71-99, 245-270: the reference's CPU path (engine/inference.py:274-278)
  int8_forward         engine/inference.py:238-272 + model/int8_blocks.py:254-298 + model/fused_blocks.py:325-363:
                       the fp16 network (stream scaled by 1/16) with int8 blocks from int8_ops, and the heads of the
                       reference's int8 network (int8_path_heads: model/fused_blocks.py:815-823, 863-874, A in fp16)
  square_feature_rows_fast  the same rows as square_feature_rows with numpy array operations (the CPU baseline's forward)

Parity of fp32_forward is pinned by the reference's own known answers (tests/test_oracle.py): the square-feature
rows of a known position (reference tests/test_model.py:166-186), grouped-query attention equal to full attention
with repeated key/value heads (:261-273), a residual-stream scale that changes no output (:125-139).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import int8_ops

NUM_SQUARES, TOKENS = 64, 70
PAWN, KNIGHT, QUEEN, KING, THEIRS, EDGE = 1, 2, 5, 6, 6, 13
NO_PIECE = 225
SLOT_ROWS = [226] * 4 + [14] * 8 + [85] * 8 + [9] + [15] * 2
ROW_OFFSETS = np.concatenate([[0], np.cumsum(SLOT_ROWS)[:-1]])
DIRECTIONS = [(0, 1), (0, -1), (1, 0), (-1, 0), (1, 1), (-1, 1), (1, -1), (-1, -1)]
KNIGHT_JUMPS = [(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)]
EPS = 1e-5


def _on_board(file: int, rank: int) -> bool:
    return 0 <= file < 8 and 0 <= rank < 8


def square_feature_rows(boards: np.ndarray) -> np.ndarray:
    """B x 64 x 23 rows within each feature's block: piece offsets (our king, their king, our queen, their queen), the 8
    neighbours' codes (13 off the board), the first piece along 8 lines and how far, attacking knights, nearest pawns up and
    down the file."""
    boards = np.asarray(boards)
    rows = np.zeros((len(boards), NUM_SQUARES, 23), dtype=np.int64)
    for b, board in enumerate(boards):
        squares = board[:NUM_SQUARES]
        firsts = {}
        for code in (KING, KING + THEIRS, QUEEN, QUEEN + THEIRS):
            where = np.nonzero(squares == code)[0]
            firsts[code] = int(where[0]) if len(where) else None
        for s in range(NUM_SQUARES):
            file, rank = s % 8, s // 8
            out = rows[b, s]
            for slot, code in enumerate((KING, KING + THEIRS, QUEEN, QUEEN + THEIRS)):
                p = firsts[code]
                out[slot] = NO_PIECE if p is None else (rank - p // 8 + 7) * 15 + file - p % 8 + 7
            for d, (df, dr) in enumerate(DIRECTIONS):
                out[4 + d] = squares[(rank + dr) * 8 + file + df] if _on_board(file + df, rank + dr) else EDGE
                out[12 + d] = 0
                for k in range(1, 8):
                    f, r = file + df * k, rank + dr * k
                    if not _on_board(f, r):
                        break
                    code = squares[r * 8 + f]
                    if code != 0:
                        out[12 + d] = 1 + (code - 1) * 7 + (k - 1)
                        break
            ours = theirs = 0
            for df, dr in KNIGHT_JUMPS:
                if _on_board(file + df, rank + dr):
                    code = squares[(rank + dr) * 8 + file + df]
                    ours += code == KNIGHT
                    theirs += code == KNIGHT + THEIRS
            out[20] = min(ours, 2) * 3 + min(theirs, 2)
            for slot, dr in enumerate((1, -1)):
                out[21 + slot] = 0
                for k in range(1, 8):
                    if not _on_board(file, rank + dr * k):
                        break
                    code = squares[(rank + dr * k) * 8 + file]
                    if code in (PAWN, PAWN + THEIRS):
                        out[21 + slot] = 1 + (code == PAWN + THEIRS) * 7 + (k - 1)
                        break
    return rows


def _board_tables():
    """Per square: its 8 neighbours, its 8 rays of 7 squares (nearest first) and its 8 knight jumps, 64 standing for off the
    board; and each square's rank and file."""
    step = lambda s, df, dr: (s // 8 + dr) * 8 + s % 8 + df if _on_board(s % 8 + df, s // 8 + dr) else 64
    rays = np.array([[[step(s, df * k, dr * k) for k in range(1, 8)] for df, dr in DIRECTIONS] for s in range(NUM_SQUARES)])
    jumps = np.array([[step(s, df, dr) for df, dr in KNIGHT_JUMPS] for s in range(NUM_SQUARES)])
    return rays, jumps, np.arange(NUM_SQUARES) // 8, np.arange(NUM_SQUARES) % 8


RAYS, JUMPS, RANKS, FILES = _board_tables()


def _first(found: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Over the last axis: whether found holds anywhere, and the first place it does (0 if nowhere)."""
    return found.any(-1), found.argmax(-1)


def square_feature_rows_fast(boards: np.ndarray) -> np.ndarray:
    """square_feature_rows for many boards at once, with numpy array operations (the CPU baseline's forward); the same rows
    (tests/test_oracle.py checks the two against each other)."""
    squares = np.asarray(boards)[:, :NUM_SQUARES].astype(np.int64)
    B = len(squares)
    padded = np.concatenate([squares, np.full((B, 1), EDGE)], 1)
    rows = np.zeros((B, NUM_SQUARES, 23), dtype=np.int64)
    for slot, code in enumerate((KING, KING + THEIRS, QUEEN, QUEEN + THEIRS)):
        present, where = _first(squares == code)
        offset = (RANKS[None, :] - RANKS[where][:, None] + 7) * 15 + FILES[None, :] - FILES[where][:, None] + 7
        rows[..., slot] = np.where(present[:, None], offset, NO_PIECE)
    along = padded[:, RAYS]                                       # B x 64 x 8 x 7
    rows[..., 4:12] = along[..., 0]
    present, where = _first((along != 0) & (along != EDGE))
    first = np.take_along_axis(along, where[..., None], -1)[..., 0]
    rows[..., 12:20] = np.where(present, 1 + (first - 1) * 7 + where, 0)
    jumps = padded[:, JUMPS]
    rows[..., 20] = np.minimum((jumps == KNIGHT).sum(-1), 2) * 3 + np.minimum((jumps == KNIGHT + THEIRS).sum(-1), 2)
    for slot, direction in ((21, 0), (22, 1)):                     # up and down the file: the first pawn, past any piece
        file_ray = along[:, :, direction]
        present, where = _first((file_ray == PAWN) | (file_ray == PAWN + THEIRS))
        pawn = np.take_along_axis(file_ray, where[..., None], -1)[..., 0]
        rows[..., slot] = np.where(present, 1 + (pawn == PAWN + THEIRS) * 7 + where, 0)
    return rows


def _tensor(state: dict, name: str, dtype=torch.float64) -> torch.Tensor:
    return state[name].detach().cpu().to(dtype)


def _rms(x: torch.Tensor, gain: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * gain


def _layers(state: dict) -> int:
    return 1 + max(int(name.split(".")[1]) for name in state if name.startswith("encoder."))


def _embedding(state: dict, boards: torch.Tensor, dtype) -> torch.Tensor:
    features = torch.from_numpy(square_feature_rows_fast(boards.numpy()) + ROW_OFFSETS)
    table = _tensor(state, "square_features.table", dtype)
    summed = table[features].sum(-2)
    embed = _tensor(state, "embed.weight", dtype)[boards] + _tensor(state, "position_embed", dtype)
    embed[:, :NUM_SQUARES] += summed
    return embed


def _heads(state: dict, output: torch.Tensor, settings: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """model/model.py:255-268 in float64: from x to bilinear logits gathered to the 1968 moves, promotions added, the value head."""
    from_squares, to_squares = state["from_squares"].cpu(), state["to_squares"].cpu()
    promotion_ids, promotion_to, promotion_pieces = (state[n].cpu() for n in ("promotion_move_ids", "promotion_to_squares", "promotion_pieces"))
    squares = output[:, :NUM_SQUARES]
    linear = lambda x, name: x @ _tensor(state, f"{name}.weight").T + _tensor(state, f"{name}.bias")
    from_vector, to_vector = linear(squares, "from_projection"), linear(squares, "to_projection")
    promotions = linear(squares, "promotion_projection")
    logits = (from_vector @ to_vector.transpose(1, 2)) / math.sqrt(output.shape[-1])
    moves = logits[:, from_squares, to_squares]
    moves[:, promotion_ids] += promotions[:, promotion_to, promotion_pieces]
    compressed = F.gelu(linear(output, "board_down_project.0")).reshape(len(output), -1)
    value = linear(F.gelu(linear(compressed, "eval_head.0")), "eval_head.2")
    return moves, value


def int8_path_heads(state: dict, output: torch.Tensor, settings: dict) -> tuple[torch.Tensor, torch.Tensor]:
    """The heads of the reference's int8 network (model/fused_blocks.py:863-874, the heads without fused ends, with the
    weights of head_weights, :815-823), in float64 from the final norm's fp16 rows: the from x to bilinear form expanded as
    (W_f x + b_f) . (W_t y + b_t) / sqrt(d) = (x A + a_bias) . y + s(x) with A = W_f^T W_t / sqrt(d) rounded to fp16 and
    a_bias = W_t^T b_f / sqrt(d), s(x) = x . (W_f^T b_t) / sqrt(d) + b_f . b_t / sqrt(d), and the narrow products (s, the
    promotion logits, board_down's inputs) from f32 weights; then the moves gathered, the promotions added, the value head."""
    d = output.shape[-1]
    scale = 1 / math.sqrt(d)
    w = lambda name: _tensor(state, name)
    from_weight, from_bias, to_weight, to_bias = w("from_projection.weight"), w("from_projection.bias"), w("to_projection.weight"), w("to_projection.bias")
    A = (from_weight.T @ to_weight * scale).half().double()
    a_bias = (to_weight.T @ from_bias * scale).float().double()
    narrow_weight = torch.cat([(to_bias @ from_weight)[None] * scale, w("promotion_projection.weight"), w("board_down_project.0.weight")]).float().double()
    narrow_bias = torch.cat([(from_bias @ to_bias)[None] * scale, w("promotion_projection.bias"), w("board_down_project.0.bias")]).float().double()
    a = output @ A + a_bias
    narrow = output @ narrow_weight.T + narrow_bias
    squares = output[:, :NUM_SQUARES]
    logits = a[:, :NUM_SQUARES] @ squares.transpose(1, 2) + narrow[:, :NUM_SQUARES, :1]
    from_squares, to_squares = state["from_squares"].cpu(), state["to_squares"].cpu()
    promotion_ids, promotion_to, promotion_pieces = (state[n].cpu() for n in ("promotion_move_ids", "promotion_to_squares", "promotion_pieces"))
    moves = logits[:, from_squares, to_squares]
    promotions = narrow[:, :NUM_SQUARES, 1:1 + w("promotion_projection.weight").shape[0]]
    moves[:, promotion_ids] += promotions[:, promotion_to, promotion_pieces]
    compressed = F.gelu(narrow[..., 1 + promotions.shape[-1]:]).reshape(len(output), -1)
    value = F.gelu(compressed @ w("eval_head.0.weight").T + w("eval_head.0.bias")) @ w("eval_head.2.weight").T + w("eval_head.2.bias")
    return moves, value


def _attention(state: dict, prefix: str, normed: torch.Tensor, templates: torch.Tensor, heads: int, eps: float = EPS) -> torch.Tensor:
    B, T, d = normed.shape
    dtype = normed.dtype
    w = lambda name: _tensor(state, f"{prefix}.{name}", dtype)
    linear = lambda name: normed @ w(f"{name}.weight").T + w(f"{name}.bias")
    q, k, v = linear("Q"), linear("K"), linear("V")
    dq = q.shape[-1] // heads
    kv_heads = k.shape[-1] // dq
    dv = v.shape[-1] // kv_heads
    q = _rms(q.reshape(B, T, heads, dq), w("q_norm.weight"), eps).transpose(1, 2)
    k = _rms(k.reshape(B, T, kv_heads, dq), w("k_norm.weight"), eps).transpose(1, 2)
    v = v.reshape(B, T, kv_heads, dv).transpose(1, 2)
    per_kv = heads // kv_heads
    k, v = k.repeat_interleave(per_kv, 1), v.repeat_interleave(per_kv, 1)
    scores = q @ k.transpose(-2, -1) / math.sqrt(dq)
    count = templates.shape[0]
    mix = normed[:, :NUM_SQUARES] @ w("template_mix.weight").T + w("template_mix.bias")
    bias = torch.einsum("biht,tij->bhij", mix.reshape(B, NUM_SQUARES, heads, count), templates.to(dtype))
    scores[:, :, :NUM_SQUARES, :NUM_SQUARES] += bias
    return (torch.softmax(scores, -1) @ v).transpose(1, 2).reshape(B, T, heads * dv)


@torch.no_grad()
def fp32_forward(state: dict, settings: dict, boards: torch.Tensor, dtype=torch.float32, eps: float = EPS) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference model's forward (model/model.py:245-270) on the CPU: (move logits B x 1968, value logits B x bins);
    eps is every RMSNorm's (the model's is 1e-5)."""
    boards = boards.cpu().long()
    heads = settings.get("n_heads", 4)
    embed = _embedding(state, boards, torch.float64).to(dtype)
    original = embed
    x = embed
    templates = _tensor(state, "templates", dtype)
    for layer in range(_layers(state)):
        p = f"encoder.{layer}"
        t = lambda name: _tensor(state, f"{p}.{name}", dtype)
        residual = t("residual_scale") * x + t("input_scale") * original
        normed = _rms(residual, t("ln1.weight"), eps)
        attended = _attention(state, p, normed, templates, heads, eps)
        residual = residual + attended @ t("combine_heads.weight").T + t("combine_heads.bias")
        hidden = _rms(residual, t("ln2.weight"), eps)
        gate, up = hidden @ t("mlp.gate_projection.weight").T, hidden @ t("mlp.up_projection.weight").T
        x = residual + (F.silu(gate) * up) @ t("mlp.down_projection.weight").T
    output = _rms(x, _tensor(state, "ln.weight", dtype), eps).double()
    moves, value = _heads(state, output, settings)
    return moves.float(), value.float()


def _fp16_state(state: dict, residual_scale: float) -> dict:
    """half_except_heads(fp16) after scale_residual_stream(residual_scale) (model/model.py:224-243)."""
    out = {}
    heads = ("from_projection", "to_projection", "promotion_projection", "board_down_project", "eval_head")
    scaled = ("embed.weight", "position_embed", "square_features.table")
    for name, value in state.items():
        value = value.detach().cpu()
        if not value.is_floating_point():
            out[name] = value
            continue
        value = value.double()
        if name in scaled or name.endswith("combine_heads.weight") or name.endswith("combine_heads.bias") or name.endswith("down_projection.weight"):
            value = value * residual_scale
        out[name] = value.float() if name.startswith(heads) else value.half()
    return out


def _np(state: dict, name: str) -> np.ndarray:
    return state[name].numpy()


def int8_block_arrays(half: dict, layer: int, weights: dict, output_scale: float, heads: int) -> dict:
    """The buffers an Int8Block holds (model/int8_blocks.py:256-272), as numpy arrays."""
    p = f"encoder.{layer}"
    dq = half[f"{p}.Q.weight"].shape[0] // heads
    kv_heads = half[f"{p}.K.weight"].shape[0] // dq
    dv = half[f"{p}.V.weight"].shape[0] // kv_heads
    block = {"eps": EPS, "heads": heads, "kv_heads": kv_heads, "dq": dq, "dv": dv, "templates_count": half[f"{p}.template_mix.weight"].shape[0] // heads,
             "ln1": _np(half, f"{p}.ln1.weight"), "ln2": _np(half, f"{p}.ln2.weight"),
             "residual_scale": _np(half, f"{p}.residual_scale"), "input_scale": _np(half, f"{p}.input_scale"),
             "q_gain": _np(half, f"{p}.q_norm.weight"), "k_gain": _np(half, f"{p}.k_norm.weight"),
             "projection_bias": np.concatenate([_np(half, f"{p}.{n}.bias") for n in ("Q", "K", "V", "template_mix")]),
             "combine_heads": _np(half, f"{p}.combine_heads.weight").T.copy(), "combine_heads_bias": _np(half, f"{p}.combine_heads.bias")}
    for name, (integers, scale) in weights[layer].items():
        block[name] = np.asarray(integers.numpy() if hasattr(integers, "numpy") else integers)
        scale = np.asarray(scale.numpy() if hasattr(scale, "numpy") else scale, dtype=np.float32)
        block[f"{name}_scale"] = (scale.astype(np.float64) * output_scale).astype(np.float32) if name == "down" else scale
    return block


def _fp16_block(half: dict, layer: int, x: np.ndarray, templates: np.ndarray, original: np.ndarray, heads: int, input_mixed: bool,
                next_scales) -> np.ndarray:
    """model/fused_blocks.py:345-354: the fp16 block with f32-summed fp16 matmuls (oracle linear) and fp16 norms."""
    p = f"encoder.{layer}"
    a = lambda name: _np(half, f"{p}.{name}")
    if not input_mixed:
        x = int8_ops.mix_in_fp16_steps(x, original, a("residual_scale"), a("input_scale"))
    norm = lambda v, gain: (_rms(torch.from_numpy(v.astype(np.float64)), torch.from_numpy(gain.astype(np.float64)))).numpy().astype(np.float16)
    projection = np.concatenate([a(f"{n}.weight") for n in ("Q", "K", "V", "template_mix")]).T
    bias = np.concatenate([a(f"{n}.bias") for n in ("Q", "K", "V", "template_mix")])
    projected = int8_ops.linear(norm(x, a("ln1.weight")), projection, bias)
    dq = a("Q.weight").shape[0] // heads
    kv_heads = a("K.weight").shape[0] // dq
    dv = a("V.weight").shape[0] // kv_heads
    attended = int8_ops.template_attention(projected, templates, a("q_norm.weight"), a("k_norm.weight"), heads, kv_heads, dq, dv,
                                           a("template_mix.weight").shape[0] // heads, EPS).astype(np.float16)
    x = int8_ops.linear(attended, a("combine_heads.weight").T, a("combine_heads.bias"), residual=x)
    gate_up = np.concatenate([a("mlp.gate_projection.weight"), a("mlp.up_projection.weight")]).T
    hidden = int8_ops.linear(norm(x, a("ln2.weight")), gate_up, gated=True)
    down = a("mlp.down_projection.weight").T
    if next_scales is None:
        return int8_ops.linear(hidden, down, residual=x)
    return int8_ops.linear(hidden, down, residual=x, original=original, residual_scale=next_scales[0], input_scale=next_scales[1])


def input_embedding(boards: np.ndarray, embed: np.ndarray, position: np.ndarray, table: np.ndarray) -> np.ndarray:
    """fp16 B x T x D: f16((f32(embed[code]) + f32(position[t])) + f32(f16(features))), features the square's 23 rows summed in f32
    one after another in slot order (model/fused_blocks.py:383-393 of the reference: store_embedding and the kernel's loop)."""
    boards = np.asarray(boards).astype(np.int64)
    rows = square_feature_rows(boards) + ROW_OFFSETS
    table = np.asarray(table, dtype=np.float16).astype(np.float32)
    features = np.zeros((len(boards), NUM_SQUARES, table.shape[1]), dtype=np.float32)
    for slot in range(rows.shape[-1]):
        features = features + table[rows[..., slot]]
    total = np.asarray(embed, dtype=np.float16).astype(np.float32)[boards] + np.asarray(position, dtype=np.float16).astype(np.float32)[:boards.shape[1]]
    total[:, :NUM_SQUARES] = total[:, :NUM_SQUARES] + features.astype(np.float16).astype(np.float32)
    return total.astype(np.float16)


@torch.no_grad()
def int8_forward(state: dict, settings: dict, weights: dict, boards: torch.Tensor, output_scale: float = 1 / 16) -> tuple[torch.Tensor, torch.Tensor]:
    """The int8 network (engine/inference.py:267-272): the layers in weights as Int8Blocks, the rest fp16 blocks, input mixes linked
    between blocks of one kind (model/fused_blocks.py:358-363); the embedding summed as the input_embedding kernel does, the final
    norm in fp16, the heads in fp32. Returns (move logits, value logits)."""
    heads = settings.get("n_heads", 4)
    boards = boards.cpu().long()
    half = _fp16_state(state, output_scale)
    x = original = input_embedding(boards.numpy(), _np(half, "embed.weight"), _np(half, "position_embed"), _np(half, "square_features.table"))
    templates = _np(half, "templates")
    kinds = ["int8" if layer in weights else "fp16" for layer in range(_layers(state))]
    for layer, kind in enumerate(kinds):
        input_mixed = layer > 0 and kinds[layer - 1] == kind
        following = layer + 1 < len(kinds) and kinds[layer + 1] == kind
        next_scales = (_np(half, f"encoder.{layer + 1}.residual_scale"), _np(half, f"encoder.{layer + 1}.input_scale")) if following else None
        if kind == "int8":
            block = int8_block_arrays(half, layer, weights, output_scale, heads)
            x = int8_ops.int8_block_forward(x, templates, original, block, input_mixed, next_scales)
        else:
            x = _fp16_block(half, layer, x, templates, original, heads, input_mixed, next_scales)
    output = _rms(torch.from_numpy(x.astype(np.float64)), half["ln.weight"].double()).half().double()
    return tuple(t.float() for t in int8_path_heads(state, output, settings))
