"""chess_value_head_no_alloc -- the value head whose hidden layer goes through the library's own device array instead of a
workspace argument -- against chess_value_head with a workspace, through the C ABI: the same answer rows and value logits to
the bit, on two calls in a row (the second smaller, so that it reuses what the first left in the array), and sizes past
the array refused before anything launches."""
import numpy as np
import pytest
import torch

from model import hip_kernels

pytestmark = pytest.mark.gpu

WIDTH, MOVES, K, H, BINS = 1969, 1968, 70 * 16, 512, 128


def inputs(B: int, seed: int, device):
    generator = torch.Generator().manual_seed(seed)
    normal = lambda *shape, std=1.0: (torch.randn(*shape, generator=generator) * std).to(device)
    return (torch.nn.functional.gelu(normal(B, K)), normal(H, K, std=0.03), normal(H, std=0.02), normal(BINS, H, std=0.05), normal(BINS, std=0.02),
            (torch.arange(BINS, dtype=torch.float32) + 0.5).div(BINS).to(device))


def call(library, entry: str, operands, B: int, device):
    c, w1, b1, w2, b2, centres = operands
    rows = torch.full((B, WIDTH), float("nan"), device=device)
    logits = torch.full((B, BINS), float("nan"), device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    pointers = [t.data_ptr() for t in (c, w1, b1, w2, b2, centres, logits, rows)]
    if entry == "workspace":
        workspace = torch.empty(B * H, device=device)
        code = library.chess_value_head(*pointers, workspace.data_ptr(), workspace.numel() * 4, B, K, H, BINS, WIDTH, MOVES, stream)
    else:
        code = library.chess_value_head_no_alloc(*pointers, B, K, H, BINS, WIDTH, MOVES, stream)
    assert code == 0, library.chess_last_error()
    torch.cuda.synchronize(device)
    return rows[:, MOVES].cpu(), logits.cpu()


def test_the_no_alloc_value_head_gives_the_workspace_calls_bits(device):
    library = hip_kernels.library_for(device)
    for B, seed in ((1024, 1), (37, 2)):
        operands = inputs(B, seed, device)
        expected_scores, expected_logits = call(library, "workspace", operands, B, device)
        scores, logits = call(library, "no_alloc", operands, B, device)
        assert not torch.isnan(expected_scores).any() and not torch.isnan(expected_logits).any()
        assert np.array_equal(scores.numpy().view(np.uint32), expected_scores.numpy().view(np.uint32))
        assert np.array_equal(logits.numpy().view(np.uint32), expected_logits.numpy().view(np.uint32))
    # past the array (4,096 positions at 512 units): refused before any launch
    operands = inputs(4, 3, device)
    pointers = [t.data_ptr() for t in operands] + [0, operands[0].data_ptr()]
    assert library.chess_value_head_no_alloc(*pointers, 4097, K, H, BINS, WIDTH, MOVES, None) == hip_kernels.UNSUPPORTED
    assert b"4097" in library.chess_last_error()
