"""The seeded legal positions the GPU tests and the benchmark evaluate (tests/golden/positions.npz), and the move generator
and token encoder that made them (tests/golden/chess_rules.py), pinned by the published perft counts of five standard
positions and by the reference's own encoding known answers (tests/test_board_encoding.py:33-230 of the reference, its
SAN move lists written here as the same moves in UCI)."""
import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
from chess_rules import START_FEN, Position, perft, play_uci, random_position  # noqa: E402

BLACK_TO_MOVE, WHITE_TO_MOVE = 13, 14
NO_CASTLING_RIGHT, CASTLING_RIGHT = 15, 16
NO_EN_PASSANT = 17
TURN_INDEX, EN_PASSANT_INDEX = 64, 69

# perft counts published for these positions (the start position, "Kiwipete" and positions 3, 4 and 5 of the standard
# perft suite): castling through and out of check, en passant with a discovered check, promotions with capture
PERFT = [
    (START_FEN, [20, 400, 8902, 197281]),
    ("r3k2r/p1ppqpb1/bn2pnp1/3PN3/1p2P3/2N2Q1p/PPPBBPPP/R3K2R w KQkq - 0 1", [48, 2039, 97862]),
    ("8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1", [14, 191, 2812, 43238]),
    ("r3k2r/Pppp1ppp/1b3nbN/nP6/BBP1P3/q4N2/Pp1P2PP/R2Q1RK1 w kq - 0 1", [6, 264, 9467]),
    ("rnbq1k1r/pp1Pbppp/2p5/8/2B5/8/PPP1NnPP/RNBQK2R w KQ - 1 8", [44, 1486, 62379]),
]


@pytest.mark.parametrize("fen, counts", PERFT, ids=["start", "kiwipete", "position3", "position4", "position5"])
def test_perft_counts(fen, counts):
    position = Position.from_fen(fen)
    assert [perft(position, depth) for depth in range(1, len(counts) + 1)] == counts


START_POSITION_ENCODING = ([4, 2, 3, 5, 6, 3, 2, 4] + [1] * 8 + [0] * 32 + [7] * 8 + [10, 8, 9, 11, 12, 9, 8, 10]
                           + [WHITE_TO_MOVE] + [CASTLING_RIGHT] * 4 + [NO_EN_PASSANT])
AFTER_E4_ENCODING = ([4, 2, 3, 5, 6, 3, 2, 4] + [1] * 8 + [0] * 16 + [0, 0, 0, 0, 7, 0, 0, 0] + [0] * 8 + [7, 7, 7, 7, 0, 7, 7, 7]
                     + [10, 8, 9, 11, 12, 9, 8, 10] + [BLACK_TO_MOVE] + [CASTLING_RIGHT] * 4 + [NO_EN_PASSANT])


def after(*moves: str) -> Position:
    return play_uci(Position.from_fen(START_FEN), *moves)


def test_the_start_position_and_black_to_move():
    assert after().tokens() == START_POSITION_ENCODING
    assert after("e2e4").tokens() == AFTER_E4_ENCODING


def test_the_products_start_tokens_are_the_start_position():
    from model.encoding import START_POSITION_TOKENS
    assert list(START_POSITION_TOKENS) == START_POSITION_ENCODING


def castling_flags(tokens: list[int]) -> tuple[int, ...]:
    return tuple(token - NO_CASTLING_RIGHT for token in tokens[65:69])


@pytest.mark.parametrize("moves, flags", [
    ("e2e4 e7e5 e1e2", (1, 1, 0, 0)),
    ("e2e4 e7e5 e1e2 e8e7", (0, 0, 0, 0)),
    ("h2h4 h7h5 h1h3", (1, 1, 0, 1)),
    ("a2a4 a7a5 a1a3 a8a6", (1, 0, 1, 0)),
    ("b2b3 b7b6 c1b2 c8b7 b2g7 b7g2 g7h8", (0, 1, 1, 1)),
    ("b2b3 b7b6 c1b2 c8b7 b2g7 b7g2 g7h8 g2h1", (0, 1, 0, 1)),
    ("e2e4 e7e5 g1f3 g8f6 f1c4 f8c5 e1g1", (1, 1, 0, 0)),
    ("e2e4 e7e5 g1f3 g8f6 f1c4 f8c5 e1g1 e8g8", (0, 0, 0, 0)),
    ("d2d4 d7d5 b1c3 b8c6 c1f4 c8f5 d1d2 d8d7 e1c1", (1, 1, 0, 0)),
    ("e2e4 e7e5 e1e2 e8e7 e2e1 e7e8", (0, 0, 0, 0)),
], ids=["white-king-moved", "both-kings-moved", "white-h-rook-moved", "both-a-rooks-moved", "black-h-rook-captured",
        "both-h-rooks-captured", "white-castled-kingside", "both-castled", "white-castled-queenside", "kings-returned-home"])
def test_lost_castling_rights(moves, flags):
    assert castling_flags(after(*moves.split()).tokens()) == flags


@pytest.mark.parametrize("moves, square", [
    ("h2h3 b7b5 h3h4 b5b4 a2a4", 40),                 # a3 mirrored for black: a6
    ("g2g4 a7a6 g4g5 h7h5", 47),                      # h6
    ("e2e4", 0),                                      # no capture available
    ("e2e4 e7e5 d2d4 e5d4 e4e5 d8e7 a2a3 d7d5", 0),   # the capturing pawn is pinned
    ("e2e4 a7a6 e4e5 d7d5", 43),                      # d6
    ("a2a3 e7e5 a3a4 e5e4 d2d4", 43),                 # d3 mirrored for black: d6
    ("e2e4 a7a6 e4e5 d7d5 g1f3", 0),                  # the square expires after a move
])
def test_en_passant_square(moves, square):
    assert after(*moves.split()).tokens()[EN_PASSANT_INDEX] == NO_EN_PASSANT + square


def test_en_passant_capture_removes_the_captured_pawn():
    tokens = after(*"e2e4 a7a6 e4e5 d7d5 e5d6 a6a5".split()).tokens()
    assert tokens[35] == 0 and tokens[43] == 1     # d5 empty, our pawn on d6


def test_every_piece_has_its_own_code():
    tokens = Position.from_fen("PNBRQKpn/brqk4/8/8/8/8/8/8 w - - 0 1").tokens()
    assert tokens[56:64] + tokens[48:52] == [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12]     # rank 8, then rank 7


@pytest.fixture(scope="module")
def fixture():
    data = np.load(GOLDEN / "positions.npz")
    return data["tokens"], data["plies"], int(data["seed"]), int(data["most_plies"])


def test_the_fixture_is_what_its_script_makes(fixture):
    tokens, plies, seed, most_plies = fixture
    rng = np.random.default_rng(seed)
    for index in range(48):
        position, played = random_position(rng, most_plies)
        assert played == plies[index] and position.tokens() == tokens[index].tolist()


def test_the_fixtures_positions_are_boards(fixture):
    tokens, plies, _, most_plies = fixture
    squares = tokens[:, :64]
    assert tokens.shape == (4096, 70) and tokens.dtype == np.uint8
    assert ((squares == 6).sum(1) == 1).all() and ((squares == 12).sum(1) == 1).all()
    assert (squares <= 12).all() and np.isin(tokens[:, TURN_INDEX], [BLACK_TO_MOVE, WHITE_TO_MOVE]).all()
    assert np.isin(tokens[:, 65:69], [NO_CASTLING_RIGHT, CASTLING_RIGHT]).all()
    assert ((tokens[:, EN_PASSANT_INDEX] >= NO_EN_PASSANT) & (tokens[:, EN_PASSANT_INDEX] < NO_EN_PASSANT + 64)).all()
    # pawns never stand on the first or last rank; the plies cover the range, and both sides are to move
    assert not np.isin(squares[:, :8], [1, 7]).any() and not np.isin(squares[:, 56:], [1, 7]).any()
    assert plies.min() == 0 and plies.max() == most_plies and 0.4 < (tokens[:, TURN_INDEX] == WHITE_TO_MOVE).mean() < 0.6
