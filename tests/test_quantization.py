"""engine/quantization.py on the CPU: GPTQ's closed forms (the reference's tests/test_int8.py:35-52), the weight layout
Int8Block reads, and the cache's names and folders (:580-595, 628-630)."""
from pathlib import Path

import torch

from engine import quantization
from engine.quantization import block_matrices, gptq, nearest, nearest_int8_weights
from model.int8_blocks import hadamard
from model.model import ChessTransformer


def test_gptq_without_correlated_inputs_rounds_to_nearest():
    torch.manual_seed(0)
    weight = torch.randn(40, 64, dtype=torch.float64)
    integers, scale = gptq(weight, torch.diag(torch.rand(64, dtype=torch.float64) + 0.5))
    assert torch.allclose(scale.double(), weight.abs().amax(dim=1) / 127, rtol=1e-6)
    assert torch.equal(integers, (weight / scale.double()[:, None]).round().to(torch.int8))
    assert all(torch.equal(a, b) for a, b in zip(nearest(weight), (integers, scale)))


def test_gptq_beats_rounding_to_nearest_on_correlated_inputs():
    torch.manual_seed(0)
    inputs = torch.randn(2000, 8, dtype=torch.float64) @ torch.randn(8, 64, dtype=torch.float64) + 0.1 * torch.randn(2000, 64, dtype=torch.float64)
    weight = torch.randn(40, 64, dtype=torch.float64)
    integers, scale = gptq(weight, inputs.t() @ inputs)
    rounded = (weight / scale.double()[:, None]).round()
    error = lambda found: (inputs @ (found * scale.double()[:, None] - weight).t()).pow(2).sum()
    assert integers.abs().max() <= 127 and error(integers.double()) < 0.5 * error(rounded)


def test_gptq_leaves_dead_inputs_at_zero():
    torch.manual_seed(1)
    inputs = torch.randn(500, 32, dtype=torch.float64)
    inputs[:, 5] = 0
    integers, _ = gptq(torch.randn(8, 32, dtype=torch.float64), inputs.t() @ inputs)
    assert (integers[:, 5] == 0).all()


def test_the_rotated_down_weight_gives_the_same_products():
    """(x H)(W_padded H / 32)^T = x_padded W^T, H the block-diagonal Sylvester matrix (H H^T = 32 I)."""
    torch.manual_seed(0)
    model = ChessTransformer(d_model=64, num_layers=1, n_heads=2, mlp_hidden=96).double()
    projection, gate_up, down, rotation = block_matrices(model.encoder[0])
    hidden = torch.randn(10, 96, dtype=torch.float64)
    padded = torch.nn.functional.pad(hidden, (0, 128 - 96))
    assert down.shape == (64, 128) and rotation.shape == (128, 128)
    assert torch.allclose((padded @ rotation) @ down.T, hidden @ model.encoder[0].mlp.down_projection.weight.T, atol=1e-10)
    assert torch.equal(rotation[:32, :32], hadamard(32).double())
    assert projection.shape == (64 + 64 + 64 + 2 * 8, 64) and gate_up.shape == (2 * 96, 64)


def test_nearest_weights_cover_all_but_the_last_block():
    model = ChessTransformer(d_model=64, num_layers=3, n_heads=2, mlp_hidden=96)
    weights = nearest_int8_weights(model)
    assert sorted(weights) == [0, 1] and sorted(weights[0]) == ["down", "gate_up", "projection"]
    integers, scale = weights[0]["down"]
    assert integers.dtype == torch.int8 and scale.dtype == torch.float32 and integers.shape == (64, 128)


def test_the_production_cache_name(tmp_path, monkeypatch):
    monkeypatch.setattr(quantization, "CACHE", tmp_path)
    checkpoint = tmp_path / "model.pt"
    checkpoint.write_bytes(b"weights")
    assert quantization.cached_weights_path(checkpoint, 0).name.endswith("_2199eb67a639465a.pt")
    assert quantization.cached_weights_path(checkpoint, 1) != quantization.cached_weights_path(checkpoint, 0)
    monkeypatch.setattr(quantization, "DAMPENING", 2 * quantization.DAMPENING)
    assert not quantization.cached_weights_path(checkpoint, 0).name.endswith("_2199eb67a639465a.pt")


def test_without_a_home_folder_nothing_is_cached(monkeypatch):
    def no_home():
        raise RuntimeError("Could not determine home directory.")
    monkeypatch.setattr(Path, "home", no_home)
    monkeypatch.delenv(quantization.CACHE_VARIABLE, raising=False)
    assert quantization.cache_folder() is None


def test_a_named_cache_folder_is_used_whatever_the_home_folder(monkeypatch, tmp_path):
    def no_home():
        raise RuntimeError("Could not determine home directory.")
    monkeypatch.setattr(Path, "home", no_home)
    monkeypatch.setenv(quantization.CACHE_VARIABLE, str(tmp_path / "int8"))
    assert quantization.cache_folder() == tmp_path / "int8"


def test_a_cache_that_cannot_be_written_costs_nothing_but_time(tmp_path, capsys):
    (tmp_path / "file").write_text("")
    quantization.cache_weights({0: {}}, tmp_path / "file" / "cache" / "weights.pt")
    assert "not cached" in capsys.readouterr().err
    quantization.cache_weights({0: {}}, None)
    assert "no home folder" in capsys.readouterr().err
    path = tmp_path / "ok" / "weights.pt"
    quantization.cache_weights({0: {"down": (torch.zeros(2, 2, dtype=torch.int8), torch.ones(2))}}, path)
    assert torch.load(path, weights_only=True)[0]["down"][1].tolist() == [1.0, 1.0]
