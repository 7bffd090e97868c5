"""The move-id table and token layout against the reference's known answers (tests/test_board_encoding.py:262-283)."""
import pytest
import torch

from model import encoding
from model.model import ChessTransformer, mlp_hidden_width


def test_move_vocabulary_size():
    # 1456 queen-line pairs + 336 knight jumps, plus 44 promoting (from, to) pairs * 4 pieces
    assert encoding.NUM_MOVE_IDS == 1792 + 176
    assert len(set(encoding.ALL_POSSIBLE_MOVES)) == encoding.NUM_MOVE_IDS


@pytest.mark.parametrize("from_square, to_square, promotion, white, expected", [
    (0, 1, None, True, 0),                       # a1b1
    (48, 56, encoding.KNIGHT_PIECE, True, 1792),  # a7a8n
    (15, 7, encoding.QUEEN_PIECE, True, 1967),    # h2h1q
    (56, 57, None, False, 0),                     # a8b8 for black
    (8, 0, encoding.KNIGHT_PIECE, False, 1792),   # a2a1n for black
])
def test_move_id_layout(from_square, to_square, promotion, white, expected):
    assert encoding.move_id(from_square, to_square, promotion, white) == expected


def test_promotions_are_knight_bishop_rook_queen():
    pieces = [encoding.PROMOTION_PIECES[i] for i in range(4)]
    assert pieces == [0, 2, 1, 3]  # the table's order is knight, rook, bishop, queen; the pieces count knight 0 .. queen 3


def test_the_token_layout():
    assert encoding.TOKENS_PER_BOARD == 70 and encoding.BOARD_VOCAB_SIZE == 13 + 2 + 2 + 64
    assert (encoding.TURN_TOKEN_OFFSET, encoding.CASTLING_TOKEN_OFFSET, encoding.EN_PASSANT_TOKEN_OFFSET) == (13, 15, 17)


def test_the_mlp_width_is_rounded_down_to_a_multiple_of_32():
    assert mlp_hidden_width(512, 1.333) == 672
    assert mlp_hidden_width(128) == 320
    assert mlp_hidden_width(16) == 32
    assert ChessTransformer(d_model=128, num_layers=1).encoder[0].mlp.up_projection.out_features == 320


def test_the_state_dict_has_the_references_names():
    names = set(ChessTransformer(d_model=32, num_layers=1, n_heads=2).state_dict())
    for name in ("embed.weight", "position_embed", "square_features.table", "templates", "encoder.0.Q.weight", "encoder.0.template_mix.bias",
                 "encoder.0.mlp.gate_projection.weight", "encoder.0.residual_scale", "board_down_project.0.weight", "eval_head.2.bias",
                 "from_squares", "promotion_pieces", "ln.weight"):
        assert name in names, name


def test_the_square_features_of_a_known_position():
    """The reference's known answer (tests/test_model.py:166-186) for the module's own feature rows."""
    from tests.test_oracle import A1, D5, E4, KNOWN
    features = ChessTransformer(d_model=32, num_layers=1, n_heads=2).square_features.indices(torch.tensor([KNOWN]))[0]
    assert features[E4, :4].tolist() == [(3 + 7) * 15 + 7, (-4 + 7) * 15 + 7, 15 * 15, (-1 + 7) * 15 + 1 + 7]
    assert features[E4, 4:12].tolist() == [0, 0, 0, 0, 0, 5 + 6, 0, 0]
    assert features[E4, 20].item() == 3 and features[D5, 21].item() == 1 + 7 + 1
    assert features[A1, 4 + 3].item() == 13 and features[A1, 12 + 3].item() == 0
