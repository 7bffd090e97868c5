"""The host-side choices around the kernels, on the CPU: tile tables, the attention launch's (position, group) runs and
the policy head's move tables (the reference's tile_for, fused_blocks.py:183-192, and its move gathers, :869-870)."""
import math

import pytest
import torch

from model import fused_blocks
from model.encoding import NUM_SQUARES
from model.fused_blocks import groups_per_workgroup, move_places, tile_for
from model.model import ChessTransformer


def test_tile_for_takes_the_first_row_share_that_fits():
    tiles = [(4, 1), (32, 3), (math.inf, 11)]
    assert tile_for(tiles, 4 * 256, 256) == 1
    assert tile_for(tiles, 4 * 256 + 1, 256) == 3
    assert tile_for(tiles, 71680, 256) == 11


@pytest.mark.parametrize("positions", [1, 3, 16, 64, 100, 256, 1024, 4096])
@pytest.mark.parametrize("kv_heads", [8, 12])
def test_attention_runs_divide_the_pairs_and_keep_the_chip_busy(positions, kv_heads):
    pairs = positions * kv_heads
    groups = groups_per_workgroup(positions, kv_heads, 256)
    workgroups = pairs // groups
    assert pairs % groups == 0
    # at least one workgroup a compute unit when there are enough pairs; when a workgroup takes several pairs, no more
    # workgroups than the picker aims at
    assert workgroups >= min(pairs, 256)
    assert groups == 1 or workgroups <= max(256, fused_blocks.ATTENTION_WORKGROUPS, pairs // 2)


def test_attention_runs_at_the_timed_batches():
    # batch 64: 256 workgroups of 2 pairs; batch 16: one pair a workgroup; batch 1024: 1,024 workgroups of 8
    assert [groups_per_workgroup(b, 8, 256) for b in (16, 64, 1024)] == [1, 2, 8]


def test_the_move_tables_are_the_gathers_of_the_heads():
    model = ChessTransformer(d_model=64, num_layers=1, n_heads=2, mlp_hidden=64, value_bins=4)
    cells, promotions = move_places(model)
    assert cells.dtype == torch.int32 and cells.shape == model.from_squares.shape
    assert torch.equal(cells.long() // NUM_SQUARES, model.from_squares) and torch.equal(cells.long() % NUM_SQUARES, model.to_squares)
    promoting = torch.zeros_like(cells, dtype=torch.bool)
    promoting[model.promotion_move_ids] = True
    assert (promotions[~promoting] == -1).all()
    placed = promotions[model.promotion_move_ids].long()
    assert torch.equal(placed // 32, model.promotion_to_squares) and torch.equal(placed % 32, 1 + model.promotion_pieces)
