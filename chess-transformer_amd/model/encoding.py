"""The board-token and move-id layout the network is trained on (reference model/encoding.py).

A position is 70 tokens: the 64 squares' piece codes (seen from the side to move), then the turn,
four castling flags and the en-passant square (reference encoding.py:3-23). The 1968 move ids are
every queen-line or knight-jump (from, to) pair in square order, then the promotions (reference
encoding.py:25-49); the tables here are computed from the board's geometry, which gives the same
order as the reference's python-chess enumeration (pinned by tests/test_encoding.py against the
reference's known ids).
"""
from __future__ import annotations

NUM_SQUARES = 64
NUM_PIECE_TYPES = 6

TURN_INDEX = 64
WHITE_KINGSIDE_INDEX = 65
WHITE_QUEENSIDE_INDEX = 66
BLACK_KINGSIDE_INDEX = 67
BLACK_QUEENSIDE_INDEX = 68
EN_PASSANT_INDEX = 69

TOKENS_PER_BOARD = 70

NUM_PIECE_CODES = 1 + 2 * NUM_PIECE_TYPES  # 0 empty, the side to move's six, the other side's six
NUM_FLAG_VALUES = 2
TURN_TOKEN_OFFSET = NUM_PIECE_CODES
CASTLING_TOKEN_OFFSET = TURN_TOKEN_OFFSET + NUM_FLAG_VALUES
EN_PASSANT_TOKEN_OFFSET = CASTLING_TOKEN_OFFSET + NUM_FLAG_VALUES
BOARD_VOCAB_SIZE = EN_PASSANT_TOKEN_OFFSET + NUM_SQUARES

# the start position's tokens, white to move (piece codes 1-6 pawn..king of the side to move, 7-12 the other side's),
# every castling right, no en-passant square: what encode_board(chess.Board()) gives (reference encoding.py:6-23); the
# engine's graph lanes record on it (reference engine/inference.py:92-93)
START_POSITION_TOKENS = (
    (4, 2, 3, 5, 6, 3, 2, 4) + (1,) * 8 + (0,) * 32 + (7,) * 8 + (10, 8, 9, 11, 12, 9, 8, 10)
    + (TURN_TOKEN_OFFSET + 1,) + (CASTLING_TOKEN_OFFSET + 1,) * 4 + (EN_PASSANT_TOKEN_OFFSET,)
)

# python-chess piece numbers, which the promotion table is ordered and offset by
KNIGHT_PIECE, BISHOP_PIECE, ROOK_PIECE, QUEEN_PIECE = 2, 3, 4, 5
QUEEN_LINES = [(0, 1), (0, -1), (1, 0), (-1, 0), (1, 1), (-1, 1), (1, -1), (-1, -1)]
KNIGHT_STEPS = [(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)]


def square(file: int, rank: int) -> int:
    return rank * 8 + file


def _destinations(start: int) -> list[int]:
    file, rank = start % 8, start // 8
    found = set()
    for df, dr in QUEEN_LINES:
        f, r = file + df, rank + dr
        while 0 <= f < 8 and 0 <= r < 8:
            found.add(square(f, r))
            f, r = f + df, r + dr
    for df, dr in KNIGHT_STEPS:
        f, r = file + df, rank + dr
        if 0 <= f < 8 and 0 <= r < 8:
            found.add(square(f, r))
    return sorted(found)


def _all_moves() -> list[tuple[int, int, int | None]]:
    """(from, to, promotion piece or None) in id order."""
    moves = [(start, end, None) for start in range(NUM_SQUARES) for end in _destinations(start)]
    for from_rank, to_rank in ((6, 7), (1, 0)):
        for from_file in range(8):
            for to_file in range(max(from_file - 1, 0), min(from_file + 2, 8)):
                for piece in (KNIGHT_PIECE, ROOK_PIECE, BISHOP_PIECE, QUEEN_PIECE):
                    moves.append((square(from_file, from_rank), square(to_file, to_rank), piece))
    return moves


ALL_POSSIBLE_MOVES = tuple(_all_moves())
NUM_MOVE_IDS = len(ALL_POSSIBLE_MOVES)
MOVE_IDS_BY_SQUARES = {move: move_id for move_id, move in enumerate(ALL_POSSIBLE_MOVES)}
MOVE_FROM_SQUARES = tuple(move[0] for move in ALL_POSSIBLE_MOVES)
MOVE_TO_SQUARES = tuple(move[1] for move in ALL_POSSIBLE_MOVES)
PROMOTION_MOVE_IDS = tuple(move_id for move_id, move in enumerate(ALL_POSSIBLE_MOVES) if move[2] is not None)
PROMOTION_TO_SQUARES = tuple(ALL_POSSIBLE_MOVES[move_id][1] for move_id in PROMOTION_MOVE_IDS)
PROMOTION_PIECES = tuple(ALL_POSSIBLE_MOVES[move_id][2] - KNIGHT_PIECE for move_id in PROMOTION_MOVE_IDS)


def move_id(from_square: int, to_square: int, promotion: int | None, white_to_move: bool = True) -> int:
    """A move's id; black's moves are mirrored (square ^ 56) to match the board seen from the side to move."""
    flip = 0 if white_to_move else 56
    return MOVE_IDS_BY_SQUARES[from_square ^ flip, to_square ^ flip, promotion]
