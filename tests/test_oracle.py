"""Pins the CPU oracle before anything is checked against it: closed forms, brute force, library routines and the
reference's own known answers -- never the oracle's formula typed out again."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import int8_ops as oracle
from oracle import network

RNG = np.random.default_rng(0)


def test_hadamard_is_sylvesters():
    H = oracle.hadamard(32)
    assert np.array_equal(H, H.T) and set(np.unique(H)) == {-1.0, 1.0}
    assert np.array_equal(H @ H.T, 32 * np.eye(32))
    i = np.arange(32)
    popcount = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    assert np.array_equal(H, (-1.0) ** popcount)


def test_the_butterflies_are_the_hadamard_product():
    small = RNG.integers(-50, 50, size=(16, 32)).astype(np.float32)  # exact in f32 at every stage
    assert np.array_equal(oracle.fwht32(small), small @ oracle.hadamard(32))
    wide = RNG.standard_normal((64, 32)).astype(np.float32)
    assert np.allclose(oracle.fwht32(wide), wide.astype(np.float64) @ oracle.hadamard(32), rtol=0, atol=1e-5)


def test_the_sum_is_a_pairwise_tree():
    # 1e8 + 1 rounds to 1e8 in f32: pairs give 0, a running sum 1, a float64 sum 2
    values = np.array([[1e8, 1, -1e8, 1]], dtype=np.float32)
    assert oracle.pairwise_sum(values)[0] == 0.0
    exact = RNG.integers(-1000, 1000, size=(5, 300)).astype(np.float32)
    assert np.array_equal(oracle.pairwise_sum(exact), exact.astype(np.int64).sum(-1).astype(np.float32))


@pytest.mark.parametrize("D", [128, 192, 512, 768])
def test_norm_quant_rounds_the_rmsnorm(D):
    x = (RNG.standard_normal((40, D)) * 4).astype(np.float16)
    gain = (RNG.random(D) + 0.5).astype(np.float16)
    q, scale = oracle.norm_quant(x, gain, 1e-5)
    normed = F.rms_norm(torch.from_numpy(x).double(), (D,), torch.from_numpy(gain).double(), 1e-5).numpy()
    step = np.abs(normed).max(-1) / 127
    assert q.dtype == np.int8 and np.abs(q).max() == 127 and (np.abs(q).max(-1) == 127).all()
    assert np.allclose(scale, step, rtol=1e-5)
    assert (np.abs(q * scale[:, None].astype(np.float64) - normed) <= 0.501 * step[:, None]).all()


@pytest.mark.parametrize("D", [64, 96, 512])
def test_rms_norm_is_torchs_to_an_fp16_step(D):
    """The fp16 blocks' norm against torch's rms_norm in float64 (the reference's nn.RMSNorm): within one rounding of fp16,
    so a dropped eps, a wrong width or a missing gain fails; with the mix, it is the mix then the norm."""
    x = (RNG.standard_normal((40, D)) * 4).astype(np.float16)
    x[0] = 0
    gain = (RNG.random(D) + 0.5).astype(np.float16)
    mixed, normed = oracle.rms_norm(x, gain, 1e-2)
    expected = F.rms_norm(torch.from_numpy(x).double(), (D,), torch.from_numpy(gain).double(), 1e-2).numpy()
    assert mixed is None and normed.dtype == np.float16 and (normed[0] == 0).all()
    assert (np.abs(normed.astype(np.float64) - expected) <= np.spacing(np.abs(expected).astype(np.float16)).astype(np.float64)).all()
    original = RNG.standard_normal((40, D)).astype(np.float16)
    rs, is_ = np.float16(0.8), np.float16(0.5)
    mixed, normed = oracle.rms_norm(x, gain, 1e-2, original, rs, is_)
    assert np.array_equal(mixed, oracle.mix_in_fp16_steps(x, original, rs, is_))
    assert np.array_equal(normed, oracle.rms_norm(mixed, gain, 1e-2)[1])


def test_the_fp16_blocks_mix_is_torchs_three_fp16_ops():
    """The fp16 block's own mix (model/fused_blocks.py:346-347) is the reference's expression run by torch in fp16, to the
    bit; the int8 blocks' mix, rounded once, differs from it on about a third of these elements, so a single rounding in
    its place fails."""
    x = (RNG.standard_normal((64, 512)) * 3).astype(np.float16)
    original = RNG.standard_normal((64, 512)).astype(np.float16)
    rs, is_ = np.float16(0.8125), np.float16(0.3)
    mixed = oracle.mix_in_fp16_steps(x, original, rs, is_)
    expected = (torch.tensor([rs]) * torch.from_numpy(x) + torch.tensor([is_]) * torch.from_numpy(original)).numpy()
    assert expected.dtype == np.float16 and np.array_equal(mixed, expected)
    assert (mixed != oracle.mix(x, original, rs, is_)).mean() > 0.1


def test_a_zero_row_quantises_to_zero():
    q, scale = oracle.norm_quant(np.zeros((2, 64), np.float16), np.ones(64, np.float16), 1e-5)
    assert (q == 0).all() and np.allclose(scale, 1e-20 / 127)


def test_the_mix_is_the_rounded_weighted_sum():
    x = (RNG.standard_normal((8, 64))).astype(np.float16)
    original = RNG.standard_normal((8, 64)).astype(np.float16)
    mixed = oracle.mix(x, original, np.float16(0.8), np.float16(0.5))
    exact = np.float64(np.float16(0.8)) * x.astype(np.float64) + np.float64(np.float16(0.5)) * original.astype(np.float64)
    assert mixed.dtype == np.float16 and np.abs(mixed.astype(np.float64) - exact).max() <= np.abs(exact).max() * 2 ** -10


@pytest.mark.parametrize("hidden, width", [(992, 1024), (320, 384), (2048, 2048)])
def test_rotate_quant_rounds_the_rotated_rows(hidden, width):
    h = RNG.standard_normal((30, hidden)).astype(np.float16)
    q, scale = oracle.rotate_quant(h, width)
    rotation = np.kron(np.eye(width // 32), oracle.hadamard(32))
    rotated = np.pad(h.astype(np.float64), ((0, 0), (0, width - hidden))) @ rotation
    step = np.abs(rotated).max(-1) / 127
    assert q.shape == (30, width) and (q[:, -(-hidden // 32) * 32:] == 0).all()
    assert np.allclose(scale, step, rtol=1e-5)
    assert (np.abs(q * scale[:, None].astype(np.float64) - rotated) <= 0.501 * step[:, None]).all()


def test_int8_sums_are_the_integer_matmul():
    x = RNG.integers(-127, 128, size=(33, 2048)).astype(np.int8)
    w = RNG.integers(-127, 128, size=(17, 2048)).astype(np.int8)
    assert np.array_equal(oracle.int8_accumulate(x, w), x.astype(np.int64) @ w.astype(np.int64).T)


def dequantised(integers, scale):
    return integers.astype(np.float64) * scale.astype(np.float64)[:, None]


@pytest.mark.parametrize("matmul", ["projection", "gate_up", "down", "mixing down"])
def test_int8_linear_is_the_dequantised_matmul(matmul):
    """The reference's check (tests/test_int8.py:59-90), on the oracle."""
    down, gated = matmul.endswith("down"), matmul == "gate_up"
    width, depth, rows = 200, 1024 if down else 256, 140
    x = RNG.integers(-127, 128, (rows, depth)).astype(np.int8)
    x_scale = (RNG.random(rows) / 100).astype(np.float32)
    weight = RNG.integers(-127, 128, (2 * width if gated else width, depth)).astype(np.int8)
    weight_scale = (RNG.random(len(weight)) / 100).astype(np.float32)
    bias = RNG.standard_normal(width).astype(np.float16) if matmul == "projection" else None
    residual = RNG.standard_normal((rows, width)).astype(np.float16) if down else None
    mix = (RNG.standard_normal((rows, width)).astype(np.float16), np.float16(0.9), np.float16(0.3)) if matmul == "mixing down" else (None,) * 3
    out = oracle.int8_linear(x, x_scale, weight, weight_scale, bias, residual, gated, *mix)
    projected = dequantised(x, x_scale) @ dequantised(weight, weight_scale).T
    if matmul == "projection":
        expected = projected + bias
    elif gated:
        gate, up = projected[:, :width], projected[:, width:]
        expected = F.silu(torch.from_numpy(gate)).numpy() * up
    else:
        expected = projected + residual
    if mix[0] is not None:
        expected = np.float64(mix[1]) * expected.astype(np.float16) + np.float64(mix[2]) * mix[0].astype(np.float64)
    assert out.dtype == np.float16 and np.allclose(out.astype(np.float64), expected, atol=1e-3, rtol=2e-3)


def test_bf16_rounding_is_torchs():
    values = np.concatenate([RNG.standard_normal(10000).astype(np.float32) * 1e3, [np.float32(1.00390625), np.float32(-3.0078125)]])
    found = oracle.round_to(values, "bf16")
    assert np.array_equal(found, torch.from_numpy(values).to(torch.bfloat16).float().numpy())


def reference_attention(projected, templates, q_gain, k_gain, heads, kv_heads, dq, dv, count, eps):
    """The reference's fp32 formula (tests/test_attention_cuda.py:51-60)."""
    projected = torch.from_numpy(projected)
    B, T, _ = projected.shape
    q, k, v, c = projected.float().split([heads * dq, kv_heads * dq, kv_heads * dv, heads * count], dim=-1)
    q = F.rms_norm(q.reshape(B, T, heads, dq), (dq,), torch.from_numpy(q_gain).float(), eps).transpose(1, 2)
    k = F.rms_norm(k.reshape(B, T, kv_heads, dq), (dq,), torch.from_numpy(k_gain).float(), eps).transpose(1, 2).repeat_interleave(heads // kv_heads, 1)
    v = v.reshape(B, T, kv_heads, dv).transpose(1, 2).repeat_interleave(heads // kv_heads, 1)
    bias = torch.einsum("biht,tij->bhij", c[:, :64].reshape(B, 64, heads, count), torch.from_numpy(templates).float())
    scores = q @ k.transpose(-2, -1) / math.sqrt(dq) + F.pad(bias, (0, T - 64, 0, T - 64))
    return (torch.softmax(scores, -1) @ v).transpose(1, 2).reshape(B, T, heads * dv).numpy()


@pytest.mark.parametrize("heads, kv_heads, dq, dv", [(24, 12, 16, 32), (8, 8, 64, 64), (4, 2, 8, 32)])
def test_template_attention_is_the_attention_in_fp32(heads, kv_heads, dq, dv):
    projected = RNG.standard_normal((3, 70, heads * dq + kv_heads * dq + kv_heads * dv + heads * 8)).astype(np.float16)
    templates = (RNG.standard_normal((8, 64, 64)) / 2).astype(np.float16)
    q_gain, k_gain = (1 + RNG.standard_normal((2, dq)) / 10).astype(np.float16)
    arguments = (projected, templates, q_gain, k_gain, heads, kv_heads, dq, dv, 8, 1e-5)
    found = oracle.template_attention(*arguments)
    assert np.abs(found - reference_attention(*arguments)).max() < 4e-3


def test_linear_is_the_matmul():
    x = RNG.standard_normal((50, 96)).astype(np.float16)
    w = RNG.standard_normal((96, 40)).astype(np.float16)
    bias, residual = RNG.standard_normal(40).astype(np.float16), RNG.standard_normal((50, 40)).astype(np.float16)
    expected = torch.from_numpy(x).double() @ torch.from_numpy(w).double() + torch.from_numpy(bias).double() + torch.from_numpy(residual).double()
    assert np.allclose(oracle.linear(x, w, bias, residual).astype(np.float64), expected.numpy(), atol=1e-2, rtol=1e-3)
    assert oracle.linear(x, w, accumulate_fp32=True).dtype == np.float32


def test_linears_input_mix_rounds_the_stream_then_weighs_it():
    """The mix branch of linear (the reference's linear_epilogue MIX, fused_blocks.py:221-224: the stream rounded to the
    output type, then residual_scale * stream + input_scale * original) through cases that fix its answer exactly: with
    the input scale 0 it is the unmixed output, with the residual scale 0 the original itself, and with scales 1 and -1
    and the original set to the rounded stream it is exactly 0, which fails a dropped term, swapped scales, a wrong sign
    or a stream mixed before its rounding."""
    x = RNG.standard_normal((30, 64)).astype(np.float16)
    w = (RNG.standard_normal((64, 48)) / 8).astype(np.float16)
    residual, original = RNG.standard_normal((30, 48)).astype(np.float16), RNG.standard_normal((30, 48)).astype(np.float16)
    one, zero = np.float16(1), np.float16(0)
    stream = oracle.linear(x, w, residual=residual)
    assert np.array_equal(oracle.linear(x, w, residual=residual, original=original, residual_scale=one, input_scale=zero), stream)
    assert np.array_equal(oracle.linear(x, w, residual=residual, original=original, residual_scale=zero, input_scale=one), original)
    unrounded = torch.from_numpy(x).double() @ torch.from_numpy(w).double() + torch.from_numpy(residual).double()
    assert (unrounded.numpy() != stream.astype(np.float64)).mean() > 0.9     # the rounding is there to be seen
    cancelled = oracle.linear(x, w, residual=residual, original=stream, residual_scale=one, input_scale=np.float16(-1))
    assert not cancelled.any()
    halves = oracle.linear(x, w, residual=residual, original=stream, residual_scale=np.float16(0.5), input_scale=np.float16(0.5))
    assert np.array_equal(halves, stream)


# white to move, so the board is not mirrored: 4k3/3p4/8/3q4/8/2N5/4P3/R3K3 w - - 0 1 (reference tests/test_model.py:166-186)
KNOWN = [0] * 64
for _square, _code in {60: 12, 51: 7, 35: 11, 18: 2, 12: 1, 0: 4, 4: 6}.items():
    KNOWN[_square] = _code
KNOWN += [14, 15, 15, 15, 15, 17]
E4, D5, A1 = 28, 35, 0


def test_the_square_features_of_a_known_position():
    features = network.square_feature_rows(np.array([KNOWN]))[0]
    assert features[E4, :4].tolist() == [(3 + 7) * 15 + 7, (-4 + 7) * 15 + 7, 15 * 15, (-1 + 7) * 15 + 1 + 7]
    assert features[E4, 4:12].tolist() == [0, 0, 0, 0, 0, 5 + 6, 0, 0]
    king, pawn, queen = 1 + (6 + 6 - 1) * 7 + 3, 1 + (1 - 1) * 7 + 1, 1 + (5 + 6 - 1) * 7 + 0
    assert features[E4, 12:20].tolist() == [king, pawn, 0, 0, 0, queen, 0, 0]
    assert features[E4, 20] == 3
    assert features[E4, 21:23].tolist() == [0, 1 + 1]
    assert features[D5, 21] == 1 + 7 + 1
    assert features[A1, 4 + 3] == 13 and features[A1, 12 + 3] == 0


def test_the_fast_square_features_are_the_square_by_square_walk():
    """The array form the CPU forward uses against the square-by-square walk that the known position pins, on boards with
    every code anywhere (several kings or none, pawns on the edge ranks) and on the known position."""
    generator = np.random.default_rng(5)
    boards = generator.integers(0, 13, (300, 70))
    boards[:40, :64] = generator.choice([0, 0, 0, 1, 7, 2, 8, 5, 11], (40, 64))
    boards[40] = KNOWN
    assert np.array_equal(network.square_feature_rows_fast(boards), network.square_feature_rows(boards))


def test_the_input_embedding_is_the_models():
    """The slot-order f32 sum of the feature rows, rounded to fp16, plus the token and position embeddings: the model's embedding in
    f64 (model/model.py:245-250 of the reference) to within the fp16 roundings."""
    model = small_state({"d_model": 64, "num_layers": 1, "n_heads": 4})
    boards = random_boards(6, seed=3)
    boards[0] = torch.tensor(KNOWN)
    with torch.no_grad():
        model.embed.weight.normal_()
        model.position_embed.normal_()
        double = model.double()
        expected = (double.embed(boards) + double.position_embed + F.pad(double.square_features(boards), (0, 0, 0, 6))).numpy()
    half = {name: value.half().numpy() for name, value in model.state_dict().items()}
    found = network.input_embedding(boards.numpy(), half["embed.weight"], half["position_embed"], half["square_features.table"])
    assert found.dtype == np.float16
    assert np.allclose(found.astype(np.float64), expected, atol=4e-3, rtol=4e-3)
    # one row changed by a known amount moves exactly the squares that use it
    table = half["square_features.table"].copy()
    row = network.square_feature_rows(boards.numpy()[:1])[0, E4, 20] + network.ROW_OFFSETS[20]
    table[row] = 0
    moved = network.input_embedding(boards.numpy()[:1], half["embed.weight"], half["position_embed"], table)
    uses = (network.square_feature_rows(boards.numpy()[:1])[0] + network.ROW_OFFSETS == row).any(-1)
    changed = (moved[0] != found[0]).any(-1)
    assert changed[:64][~uses].sum() == 0 and changed[E4]


def small_state(settings, seed=0):
    from model.model import ChessTransformer
    torch.manual_seed(seed)
    model = ChessTransformer(**settings).eval()
    with torch.no_grad():
        for block in model.encoder:
            block.residual_scale.fill_(0.8)
            block.input_scale.fill_(0.5)
        model.templates.normal_()
        model.square_features.table.normal_(std=0.1)
        model.from_projection.weight.mul_(8)
    return model


SMALL = {"d_model": 128, "num_layers": 3, "n_heads": 4, "kv_heads": 2, "qk_ratio": [0.25, 0.5, 0.75], "mlp_hidden": 320, "value_bins": 16}


def random_boards(count, seed=0):
    generator = torch.Generator().manual_seed(seed)
    boards = torch.randint(0, 13, (count, 70), generator=generator)
    boards[:, 64:] = torch.tensor([14, 16, 16, 16, 16, 17])
    return boards


def test_grouped_query_attention_is_heads_sharing_their_keys_and_values():
    """The reference's check (tests/test_model.py:261-273) on the oracle's forward."""
    settings = {"d_model": 32, "num_layers": 2, "n_heads": 4, "kv_heads": 2}
    grouped = small_state(settings).state_dict()
    full = dict(grouped)
    for name in [f"encoder.{block}.{projection}.{kind}" for block in range(2) for projection in "KV" for kind in ("weight", "bias")]:
        full[name] = grouped[name].reshape(2, 8, *grouped[name].shape[1:]).repeat_interleave(2, dim=0).flatten(0, 1)
    boards = random_boards(4)
    for a, b in zip(network.fp32_forward(grouped, settings, boards), network.fp32_forward(full, settings, boards)):
        assert torch.allclose(a, b, atol=1e-5)


def test_scaling_the_residual_stream_changes_no_output():
    """The reference's check (tests/test_model.py:125-139): with the norms' eps at 0, which is all that sees the scale."""
    model = small_state(SMALL)
    boards = random_boards(3)
    before = network.fp32_forward({k: v.clone() for k, v in model.state_dict().items()}, SMALL, boards, eps=0.0)
    after = network.fp32_forward(model.scale_residual_stream(1 / 16).state_dict(), SMALL, boards, eps=0.0)
    assert all(torch.allclose(a, b, atol=1e-4) for a, b in zip(before, after))


def test_a_block_with_uniform_attention_adds_the_mean_value_row():
    """A closed form of one block: with Q's and K's weights and biases zero and no template bias the scores are all equal, so
    every token attends to the mean of the 70 value rows; with the mlp's down weight zero and the input unmixed (residual
    scale 1, input scale 0) the block adds combine_heads(mean V) to its input. The oracle's forward of such a one-block
    model equals the heads of the final norm of embedding + that row, computed here from the state alone."""
    settings = {"d_model": 32, "num_layers": 1, "n_heads": 4, "kv_heads": 2, "value_bins": 8}
    state = {name: value.double() if value.is_floating_point() else value for name, value in small_state(settings).state_dict().items()}
    for name in ("Q.weight", "Q.bias", "K.weight", "K.bias", "template_mix.weight", "template_mix.bias", "mlp.down_projection.weight",
                 "input_scale"):
        state[f"encoder.0.{name}"] = torch.zeros_like(state[f"encoder.0.{name}"])
    state["encoder.0.residual_scale"] = torch.ones(1, dtype=torch.float64)
    boards = random_boards(3, seed=9)
    embedded = network._embedding(state, boards, torch.float64)
    rms = lambda x, gain: x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5) * gain
    values = rms(embedded, state["encoder.0.ln1.weight"]) @ state["encoder.0.V.weight"].T + state["encoder.0.V.bias"]     # B x 70 x 16
    per_head = values.reshape(3, 70, 2, 8).mean(1).repeat_interleave(2, 1).reshape(3, 1, 32)          # each head reads its group's mean
    x = embedded + per_head @ state["encoder.0.combine_heads.weight"].T + state["encoder.0.combine_heads.bias"]
    expected = network._heads(state, rms(x, state["ln.weight"]), settings)
    found = network.fp32_forward(state, settings, boards, dtype=torch.float64)
    assert all(torch.allclose(a.double(), b, atol=1e-5) for a, b in zip(found, expected))


def test_the_heads_with_identity_projections_are_dot_products_of_squares():
    """The oracle's heads with the from and to projections the identity (biases zero) and the promotion projection a known
    constant: a move's logit is x[from] . x[to] / sqrt(d), plus that constant's piece column on a promotion; a1b1 (id 0)
    and a7a8n (id 1792, knight column) checked by hand."""
    settings = {"d_model": 32, "num_layers": 1, "n_heads": 4, "value_bins": 8}
    state = {name: value.double() if value.is_floating_point() else value for name, value in small_state(settings).state_dict().items()}
    for side in ("from", "to"):
        state[f"{side}_projection.weight"], state[f"{side}_projection.bias"] = torch.eye(32, dtype=torch.float64), torch.zeros(32, dtype=torch.float64)
    state["promotion_projection.weight"] = torch.zeros(4, 32, dtype=torch.float64)
    state["promotion_projection.bias"] = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.float64)
    x = torch.randn(2, 70, 32, dtype=torch.float64)
    logits, _ = network._heads(state, x, settings)
    assert torch.allclose(logits[:, 0], (x[:, 0] * x[:, 1]).sum(-1) / math.sqrt(32))
    assert torch.allclose(logits[:, 1792], (x[:, 48] * x[:, 56]).sum(-1) / math.sqrt(32) + 1.0)


def test_the_int8_paths_heads_are_the_models_where_its_roundings_are_exact():
    """The heads of the reference's int8 network (A = W_f^T W_t / sqrt(d) in fp16, the bilinear form expanded into a, a_bias
    and the narrow terms) against the model's heads, with dyadic weights and biases for which A and every f32 weight are
    exact: then the two are the same function (a dropped term of the expansion, a transposed A or a wrong narrow column
    fails), up to float64 rounding. With other weights they differ by A's fp16 rounding only."""
    settings = {"d_model": 16, "num_layers": 1, "n_heads": 2, "value_bins": 8}
    state = {name: value.double() if value.is_floating_point() else value for name, value in small_state(settings).state_dict().items()}
    generator = torch.Generator().manual_seed(3)
    dyadic = lambda *shape: torch.randint(-8, 9, shape, generator=generator).double() / 8
    state["from_projection.weight"], state["to_projection.weight"] = 2 * torch.eye(16, dtype=torch.float64), torch.diag(dyadic(16)) * 2
    for name in ("from_projection.bias", "to_projection.bias", "promotion_projection.bias", "board_down_project.0.bias"):
        state[name] = dyadic(*state[name].shape)
    for name in ("promotion_projection.weight", "board_down_project.0.weight"):
        state[name] = dyadic(*state[name].shape)
    x = torch.randn(3, 70, 16, generator=generator).half().double()
    for found, expected in zip(network.int8_path_heads(state, x, settings), network._heads(state, x, settings)):
        assert torch.allclose(found, expected, atol=1e-12)
    state["from_projection.weight"] = torch.randn(16, 16, generator=generator, dtype=torch.float64)
    rounded, exact = network.int8_path_heads(state, x, settings)[0], network._heads(state, x, settings)[0]
    assert 0 < (rounded - exact).abs().max() < 1e-2


def test_the_oracles_forward_is_the_models():
    model = small_state(SMALL)
    boards = random_boards(5)
    with torch.no_grad():
        expected = model(boards)
    for found, want in zip(network.fp32_forward(model.state_dict(), SMALL, boards), expected):
        assert torch.allclose(found, want, atol=1e-4)


def test_the_int8_network_computes_what_the_model_does():
    """The reference's bar for its int8 model (tests/test_int8.py:359-373), for the oracle's int8 network."""
    from engine.quantization import nearest_int8_weights
    from model.model import expected_score
    model = small_state(SMALL)
    boards = random_boards(6)
    with torch.no_grad():
        logits, values = model(boards)
    found_logits, found_values = network.int8_forward(model.state_dict(), SMALL, nearest_int8_weights(model), boards)
    distance = 0.5 * (torch.softmax(found_logits, -1) - torch.softmax(logits, -1)).abs().sum(-1)
    assert distance.max() < 0.005 and torch.equal(found_logits.argmax(-1), logits.argmax(-1))
    assert torch.allclose(expected_score(found_values), expected_score(values), atol=5e-3)


def test_down_mixes_the_next_blocks_input_to_the_bit():
    """Mixing the next block's input in down's epilogue gives the bits of mixing it at the next block's start
    (the reference's tests/test_int8.py:376-387), on the oracle's blocks."""
    from engine.quantization import nearest_int8_weights
    model = small_state(SMALL)
    weights = nearest_int8_weights(model)
    half = network._fp16_state(model.state_dict(), 1 / 16)
    x = original = (torch.randn(2, 70, 128) / 16).half().numpy()
    templates = half["templates"].numpy()
    blocks = [network.int8_block_arrays(half, layer, weights, 1 / 16, 4) for layer in range(2)]
    scales = (blocks[1]["residual_scale"], blocks[1]["input_scale"])
    linked = oracle.int8_block_forward(oracle.int8_block_forward(x, templates, original, blocks[0], False, scales), templates, original, blocks[1],
                                       True)
    separate = oracle.int8_block_forward(oracle.int8_block_forward(x, templates, original, blocks[0], False), templates, original, blocks[1], False)
    assert np.array_equal(linked.view(np.uint16), separate.view(np.uint16))
