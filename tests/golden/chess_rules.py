"""Legal chess moves and the network's board tokens, for seeded random legal positions -- TEST AND BENCHMARK INPUT ONLY.

The reference draws its positions with python-chess (model/encoding.py:72-92 encodes them), which is not installed here.
This is a small move generator of this repository's own: a 64-square board of signed piece codes, pseudo-legal moves
from step and ray tables, and legality by asking whether the mover's king is attacked after the move. It is pinned by
the published perft counts of five standard positions and by the reference's own encoding known answers
(tests/test_golden_positions.py).

Squares are 0 (a1) .. 63 (h8), rank-major. A piece is +1..+6 for white's pawn, knight, bishop, rook, queen, king and
-1..-6 for black's; 0 is empty. Castling rights are the bits K=1, Q=2, k=4, q=8. The en-passant square is the square a
pawn skipped on the last move (python-chess's ep_square), or -1.
"""
from __future__ import annotations

from dataclasses import dataclass, field

PAWN, KNIGHT, BISHOP, ROOK, QUEEN, KING = 1, 2, 3, 4, 5, 6
WHITE_KINGSIDE, WHITE_QUEENSIDE, BLACK_KINGSIDE, BLACK_QUEENSIDE = 1, 2, 4, 8
START_FEN = "rnbqkbnr/pppppppp/8/8/8/8/PPPPPPPP/RNBQKBNR w KQkq - 0 1"

# the network's token layout (the reference's model/encoding.py:6-23)
TURN_TOKEN_OFFSET, CASTLING_TOKEN_OFFSET, EN_PASSANT_TOKEN_OFFSET = 13, 15, 17
PIECE_TYPES = 6


def _on_board(file: int, rank: int) -> bool:
    return 0 <= file < 8 and 0 <= rank < 8


def _steps(deltas) -> list[list[int]]:
    return [[(r + dr) * 8 + f + df for df, dr in deltas if _on_board(f + df, r + dr)] for r in range(8) for f in range(8)]


def _rays(deltas) -> list[list[list[int]]]:
    rays = []
    for square in range(64):
        f, r = square % 8, square // 8
        per_square = []
        for df, dr in deltas:
            line, nf, nr = [], f + df, r + dr
            while _on_board(nf, nr):
                line.append(nr * 8 + nf)
                nf, nr = nf + df, nr + dr
            per_square.append(line)
        rays.append(per_square)
    return rays


KNIGHT_STEPS = _steps([(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)])
KING_STEPS = _steps([(1, 0), (1, 1), (0, 1), (-1, 1), (-1, 0), (-1, -1), (0, -1), (1, -1)])
ROOK_RAYS = _rays([(1, 0), (-1, 0), (0, 1), (0, -1)])
BISHOP_RAYS = _rays([(1, 1), (-1, 1), (1, -1), (-1, -1)])
# the squares a pawn of each colour attacks from a square (index 0 white, 1 black)
PAWN_ATTACKS = (_steps([(-1, 1), (1, 1)]), _steps([(-1, -1), (1, -1)]))
# a rook leaving or being taken on its home square ends that castling right
ROOK_HOMES = {0: WHITE_QUEENSIDE, 7: WHITE_KINGSIDE, 56: BLACK_QUEENSIDE, 63: BLACK_KINGSIDE}


@dataclass(frozen=True)
class Move:
    start: int
    end: int
    promotion: int = 0          # piece type promoted to (2..5), or 0

    def uci(self) -> str:
        name = lambda s: "abcdefgh"[s % 8] + str(s // 8 + 1)
        return name(self.start) + name(self.end) + ("", "", "n", "b", "r", "q")[self.promotion]


def _pawn_moves(start: int, end: int, promote: bool) -> list[Move]:
    return [Move(start, end, piece) for piece in (QUEEN, ROOK, BISHOP, KNIGHT)] if promote else [Move(start, end)]


@dataclass
class Position:
    squares: list[int] = field(default_factory=lambda: [0] * 64)
    white: bool = True
    castling: int = 0
    en_passant: int = -1

    @staticmethod
    def from_fen(fen: str) -> "Position":
        placement, turn, castling, en_passant = fen.split()[:4]
        position = Position()
        codes = {"p": PAWN, "n": KNIGHT, "b": BISHOP, "r": ROOK, "q": QUEEN, "k": KING}
        for rank_from_top, row in enumerate(placement.split("/")):
            file = 0
            for char in row:
                if char.isdigit():
                    file += int(char)
                    continue
                piece = codes[char.lower()]
                position.squares[(7 - rank_from_top) * 8 + file] = piece if char.isupper() else -piece
                file += 1
        position.white = turn == "w"
        position.castling = sum(bit for letter, bit in zip("KQkq", (1, 2, 4, 8)) if letter in castling)
        position.en_passant = -1 if en_passant == "-" else "abcdefgh".index(en_passant[0]) + 8 * (int(en_passant[1]) - 1)
        return position

    def copy(self) -> "Position":
        return Position(self.squares[:], self.white, self.castling, self.en_passant)

    def king(self, white: bool) -> int:
        return self.squares.index(KING if white else -KING)

    def attacked(self, square: int, by_white: bool) -> bool:
        """Whether a piece of the colour by_white attacks square."""
        sign = 1 if by_white else -1
        board = self.squares
        # a pawn of that colour attacks square from the squares a pawn of the other colour would attack from square
        if any(board[s] == sign * PAWN for s in PAWN_ATTACKS[1 if by_white else 0][square]):
            return True
        if any(board[s] == sign * KNIGHT for s in KNIGHT_STEPS[square]):
            return True
        if any(board[s] == sign * KING for s in KING_STEPS[square]):
            return True
        for rays, sliders in ((ROOK_RAYS, (ROOK, QUEEN)), (BISHOP_RAYS, (BISHOP, QUEEN))):
            for ray in rays[square]:
                for s in ray:
                    piece = board[s]
                    if piece:
                        if piece * sign > 0 and abs(piece) in sliders:
                            return True
                        break
        return False

    def pseudo_legal(self) -> list[Move]:
        board, sign = self.squares, 1 if self.white else -1
        moves: list[Move] = []
        forward, home_rank, last_rank = (8, 1, 7) if self.white else (-8, 6, 0)
        for start, piece in enumerate(board):
            if piece * sign <= 0:
                continue
            kind = abs(piece)
            if kind == PAWN:
                one = start + forward
                promote = one // 8 == last_rank
                if board[one] == 0:
                    moves.extend(_pawn_moves(start, one, promote))
                    two = one + forward
                    if start // 8 == home_rank and board[two] == 0:
                        moves.append(Move(start, two))
                for target in PAWN_ATTACKS[0 if self.white else 1][start]:
                    if board[target] * sign < 0:
                        moves.extend(_pawn_moves(start, target, promote))
                    elif target == self.en_passant:
                        moves.append(Move(start, target))
            elif kind == KNIGHT or kind == KING:
                for target in (KNIGHT_STEPS if kind == KNIGHT else KING_STEPS)[start]:
                    if board[target] * sign <= 0:
                        moves.append(Move(start, target))
            else:
                rays = (BISHOP_RAYS[start] if kind == BISHOP else ROOK_RAYS[start] if kind == ROOK else BISHOP_RAYS[start] + ROOK_RAYS[start])
                for ray in rays:
                    for target in ray:
                        if board[target] * sign > 0:
                            break
                        moves.append(Move(start, target))
                        if board[target]:
                            break
        moves.extend(self._castles())
        return moves

    def _castles(self) -> list[Move]:
        board = self.squares
        if self.white:
            king, rights, enemy = 4, (WHITE_KINGSIDE, WHITE_QUEENSIDE), False
        else:
            king, rights, enemy = 60, (BLACK_KINGSIDE, BLACK_QUEENSIDE), True
        if not self.castling & (rights[0] | rights[1]) or self.attacked(king, enemy):
            return []
        castles = []
        # kingside: f and g empty and not attacked; queenside: b, c, d empty, c and d not attacked
        if self.castling & rights[0] and board[king + 1] == 0 and board[king + 2] == 0 \
                and not self.attacked(king + 1, enemy) and not self.attacked(king + 2, enemy):
            castles.append(Move(king, king + 2))
        if self.castling & rights[1] and board[king - 1] == 0 and board[king - 2] == 0 and board[king - 3] == 0 \
                and not self.attacked(king - 1, enemy) and not self.attacked(king - 2, enemy):
            castles.append(Move(king, king - 2))
        return castles

    def play(self, move: Move) -> "Position":
        """The position after move (a new Position)."""
        after = self.copy()
        board = after.squares
        piece = board[move.start]
        kind = abs(piece)
        captured_at = move.end
        if kind == PAWN and move.end == self.en_passant and board[move.end] == 0:
            captured_at = move.end - (8 if self.white else -8)
            board[captured_at] = 0
        board[move.end] = (move.promotion * (1 if piece > 0 else -1)) if move.promotion else piece
        board[move.start] = 0
        if kind == KING and abs(move.end - move.start) == 2:
            rook_from, rook_to = (move.start + 3, move.start + 1) if move.end > move.start else (move.start - 4, move.start - 1)
            board[rook_to], board[rook_from] = board[rook_from], 0
        if kind == KING:
            after.castling &= ~((WHITE_KINGSIDE | WHITE_QUEENSIDE) if piece > 0 else (BLACK_KINGSIDE | BLACK_QUEENSIDE))
        for square in (move.start, move.end):
            after.castling &= ~ROOK_HOMES.get(square, 0)
        after.en_passant = (move.start + move.end) // 2 if kind == PAWN and abs(move.end - move.start) == 16 else -1
        after.white = not self.white
        return after

    def legal(self) -> list[Move]:
        moves = []
        for move in self.pseudo_legal():
            after = self.play(move)
            if not after.attacked(after.king(self.white), not self.white):
                moves.append(move)
        return moves

    def has_legal_en_passant(self) -> bool:
        if self.en_passant < 0:
            return False
        return any(move.end == self.en_passant and abs(self.squares[move.start]) == PAWN for move in self.legal())

    def tokens(self) -> list[int]:
        """The 70 tokens the network reads (the reference's encode_board, model/encoding.py:72-92): the squares from the
        side to move (ranks flipped, square ^ 56, when black moves), its pieces 1-6 and the other side's 7-12; the turn
        (14 white, 13 black); castling rights as the mover's kingside, queenside, then the other side's (16 a right, 15
        none); the en-passant square from the mover's side when a legal capture onto it exists (17 + square), else 17."""
        flip = 0 if self.white else 56
        sign = 1 if self.white else -1
        out = [0] * 64
        for square, piece in enumerate(self.squares):
            if piece:
                out[square ^ flip] = abs(piece) if piece * sign > 0 else abs(piece) + PIECE_TYPES
        ours = (WHITE_KINGSIDE, WHITE_QUEENSIDE) if self.white else (BLACK_KINGSIDE, BLACK_QUEENSIDE)
        theirs = (BLACK_KINGSIDE, BLACK_QUEENSIDE) if self.white else (WHITE_KINGSIDE, WHITE_QUEENSIDE)
        flags = [CASTLING_TOKEN_OFFSET + bool(self.castling & bit) for bit in ours + theirs]
        en_passant = self.en_passant ^ flip if self.has_legal_en_passant() else 0
        return out + [TURN_TOKEN_OFFSET + self.white] + flags + [EN_PASSANT_TOKEN_OFFSET + en_passant]


def perft(position: Position, depth: int) -> int:
    """The number of legal move sequences of depth plies."""
    moves = position.legal()
    if depth == 1:
        return len(moves)
    return sum(perft(position.play(move), depth - 1) for move in moves)


def play_uci(position: Position, *moves: str) -> Position:
    """position after the moves in UCI (e2e4, e7e8q), each checked to be legal."""
    for text in moves:
        legal = {move.uci(): move for move in position.legal()}
        if text not in legal:
            raise ValueError(f"{text} is not legal here")
        position = position.play(legal[text])
    return position


def random_position(rng, most_plies: int = 80) -> tuple[Position, int]:
    """The start position after a uniform 0..most_plies random legal moves, each uniform among the legal moves, and the plies
    played; a game that ends sooner stops at its last position with a legal move."""
    position, played = Position.from_fen(START_FEN), 0
    for _ in range(int(rng.integers(0, most_plies + 1))):
        moves = position.legal()
        after = position.play(moves[int(rng.integers(0, len(moves)))])
        if not after.legal():
            break
        position, played = after, played + 1
    return position, played
