"""Numpy restatement of the int8 hot-path operators -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
use this module, as the checker. The product never imports it.

Declared arithmetic (shared with the HIP kernels in chess-transformer_amd/csrc):
every float step below is ONE IEEE-754 binary32 operation rounded to nearest
even -- multiply, add, subtract, divide, sqrt, rint, min/max -- and there is no
fused multiply-add anywhere (the kernels are built with -ffp-contract=off).
The one exception is the gated (SiLU) epilogue, whose sigmoid the kernel takes
from the hardware exp2/reciprocal: it is checked at the reference's tolerance.
numpy's float32 arithmetic is exactly that, so the integer and quantised
outputs here and on the GPU agree to the bit when the inputs do. Conversions
fp16/bf16 <- f32 round to nearest even; int32 -> f32 rounds to nearest even.

Where the reference leaves an order open (Triton's tl.sum, its contraction of
a*b+c into fma, tl.rsqrt, tl.sigmoid), this module fixes one; bitwise parity
with the reference's NVIDIA kernels is therefore not claimed -- the reference's
own tolerance checks are (tests/test_int8.py:76-90, 246-281 and
tests/test_attention_cuda.py:51-71 in the reference).

Pinning: tests/test_oracle.py checks every function here against closed forms
and brute force (exact int64 matmul, H H^T = 32 I, fp64 dequantised matmul,
torch's rms_norm / softmax formula of the reference tests).
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
F16 = np.float16

# model/int8_blocks.py:15-17
HADAMARD_BLOCK = 32
DOWN_INPUT_MULTIPLE = 128
INT8_MAX = 127
ABSMAX_FLOOR = F32(1e-20)  # int8_blocks.py:173, 227


def hadamard(size: int) -> np.ndarray:
    """Sylvester's +-1 Hadamard matrix (model/int8_blocks.py:54-58): entry (i, j) is (-1)^popcount(i & j)."""
    matrix = np.ones((1, 1), dtype=np.float32)
    while matrix.shape[0] < size:
        matrix = np.block([[matrix, matrix], [matrix, -matrix]])
    return matrix


def down_inputs(hidden: int) -> int:
    """model/int8_blocks.py:61-62: the mlp hidden width padded to a multiple of 128."""
    return -(-hidden // DOWN_INPUT_MULTIPLE) * DOWN_INPUT_MULTIPLE


def next_pow2(n: int) -> int:
    return 1 << max(0, (n - 1).bit_length())


def pairwise_sum(values: np.ndarray) -> np.ndarray:
    """Sum over the last axis as a balanced tree of adjacent pairs, the row zero-padded to a power of two.

    The kernels reach the same tree: a lane sums its contiguous power-of-two chunk as a tree, then the
    wavefront's xor butterfly (offsets 1, 2, 4, ...) adds the lanes' partials pairwise in lane order.
    """
    width = values.shape[-1]
    padded = next_pow2(width)
    if padded != width:
        values = np.concatenate([values, np.zeros((*values.shape[:-1], padded - width), values.dtype)], -1)
    while values.shape[-1] > 1:
        values = values[..., 0::2] + values[..., 1::2]
    return values[..., 0]


def quantize_rows(y: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-row int8 (int8_blocks.py:173-175, 227-231): absmax floored at 1e-20, q = rint(y * (127 / absmax))."""
    y = y.astype(F32, copy=False)
    absmax = np.maximum(np.abs(y).max(axis=-1), ABSMAX_FLOOR)
    inverse_step = F32(INT8_MAX) / absmax
    q = np.rint(y * inverse_step[..., None]).astype(np.int8)
    return q, absmax / F32(INT8_MAX)


def rms_normalise(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    """y = (x * (1 / sqrt(tree_sum(x*x) / D + eps))) * gain, in f32 (int8_blocks.py:171-172)."""
    x = x.astype(F32, copy=False)
    D = x.shape[-1]
    mean = pairwise_sum(x * x) / F32(D)
    inverse = F32(1.0) / np.sqrt(mean + F32(eps))
    return (x * inverse[..., None]) * gain.astype(F32)


def mix(x: np.ndarray, original: np.ndarray, residual_scale, input_scale, dtype=F16) -> np.ndarray:
    """The block's input mix, rounded to the stream's dtype: (x * rs) + (original * is) (model/model.py:73, int8_blocks.py:168)."""
    rs = F32(np.asarray(residual_scale, dtype=np.float32).reshape(-1)[0])
    is_ = F32(np.asarray(input_scale, dtype=np.float32).reshape(-1)[0])
    return round_to((x.astype(F32) * rs) + (original.astype(F32) * is_), dtype)


def mix_in_fp16_steps(x: np.ndarray, original: np.ndarray, residual_scale, input_scale) -> np.ndarray:
    """The fp16 block's own input mix (model/fused_blocks.py:346-347), three fp16 ops each rounded as torch rounds them:
    f16(f16(rs * x) + f16(is * original)), each product and the sum formed in f32 (a product of two fp16 is exact there)."""
    rs = F32(np.asarray(residual_scale, dtype=np.float16).reshape(-1)[0])
    is_ = F32(np.asarray(input_scale, dtype=np.float16).reshape(-1)[0])
    scaled = (rs * x.astype(F32)).astype(F16).astype(F32)
    added = (is_ * original.astype(F32)).astype(F16).astype(F32)
    return (scaled + added).astype(F16)


def norm_quant(x: np.ndarray, gain: np.ndarray, eps: float) -> tuple[np.ndarray, np.ndarray]:
    """model/int8_blocks.py:156-175 (MIX=0): RMSNorm with gain, then per-row int8 and its scale."""
    q, scale = quantize_rows(rms_normalise(x.reshape(-1, x.shape[-1]), gain, eps))
    return q.reshape(x.shape), scale.reshape(x.shape[:-1])


def mix_norm_quant(x, original, residual_scale, input_scale, gain, eps) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """model/int8_blocks.py:156-175 (MIX=1) and :201-207: the mixed stream (fp16) and its int8 rows."""
    mixed = mix(x, original, residual_scale, input_scale)
    q, scale = norm_quant(mixed, gain, eps)
    return mixed, q, scale


def rms_norm(x: np.ndarray, gain: np.ndarray, eps: float, original=None, residual_scale=None, input_scale=None):
    """The fp16 blocks' RMSNorm (nn.RMSNorm in fp16 at model/fused_blocks.py:348, 351 and 863), in norm_quant's f32 order
    rounded once to fp16: (mixed or None, f16(rms_normalise(mixed or x))). With original, the block's own input mix
    (:346-347) comes first, as mix_in_fp16_steps() rounds it."""
    mixed = mix_in_fp16_steps(x, original, residual_scale, input_scale) if original is not None else None
    rows = mixed if mixed is not None else x
    normed = rms_normalise(rows.reshape(-1, rows.shape[-1]), gain, eps).astype(F16)
    return mixed, normed.reshape(rows.shape)


def fwht32(rows: np.ndarray) -> np.ndarray:
    """rows[..., 32] @ hadamard(32) as five f32 butterfly stages, spans 1, 2, 4, 8, 16: (a, b) -> (a + b, a - b)."""
    out = rows.astype(F32)
    shape = out.shape
    for span in (1, 2, 4, 8, 16):
        halves = out.reshape(*shape[:-1], HADAMARD_BLOCK // (2 * span), 2, span)
        a, b = halves[..., 0, :], halves[..., 1, :]
        out = np.stack([a + b, a - b], axis=-2).reshape(shape)
    return out


def rotate_quant(h: np.ndarray, width: int) -> tuple[np.ndarray, np.ndarray]:
    """model/int8_blocks.py:216-246: h zero-padded to width, each 32 block times Sylvester H32, per-row int8."""
    if width % HADAMARD_BLOCK or width < h.shape[-1]:
        raise ValueError(f"rotate_quant pads {h.shape[-1]} columns to a width divisible by {HADAMARD_BLOCK}, not {width}")
    N = h.shape[-1]
    rows = h.reshape(-1, N)
    padded = np.zeros((rows.shape[0], width), dtype=F32)
    padded[:, :N] = rows
    rotated = fwht32(padded.reshape(rows.shape[0], width // HADAMARD_BLOCK, HADAMARD_BLOCK)).reshape(rows.shape[0], width)
    q, scale = quantize_rows(rotated)
    return q.reshape(*h.shape[:-1], width), scale.reshape(h.shape[:-1])


def int8_accumulate(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact int32 sums of x[M, K] @ w[N, K]^T. Every partial sum is an integer below 2^53, so float64 BLAS is exact."""
    return np.rint(x.astype(np.float64) @ w.astype(np.float64).T).astype(np.int64)


def silu_product(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up, the gated epilogue (int8_blocks.py:284 with linear_epilogue, fused_blocks.py:215-216), in float64:
    the kernel takes the sigmoid from the hardware's exp2 and reciprocal, so this step is a tolerance reference."""
    g = gate.astype(np.float64)
    return (g / (1.0 + np.exp(-g))) * up.astype(np.float64)


def to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit pattern (uint16), round to nearest even; NaN stays a quiet NaN."""
    bits = values.astype(F32).view(np.uint32)
    rounded = bits + (np.uint32(0x7FFF) + ((bits >> 16) & 1))
    out = (rounded >> 16).astype(np.uint16)
    nan = np.isnan(values)
    out[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(F32)


def round_to(values: np.ndarray, dtype) -> np.ndarray:
    """Round f32 values to the output dtype: np.float16, np.float32, or "bf16" (returned as f32 holding bf16 values)."""
    if dtype == "bf16":
        return from_bf16_bits(to_bf16_bits(values))
    return values.astype(dtype)


def int8_linear(x, x_scale, weight, weight_scale, bias=None, residual=None, gated=False, original=None, residual_scale=None,
                input_scale=None, out_dtype=F16) -> np.ndarray:
    """model/int8_blocks.py:66-102 with linear_epilogue (fused_blocks.py:208-225), in the op order of int8_cuda.py:146-181
    without fma contraction:
      v = f32(acc) * x_scale[m];  out = v * w_scale[n];  [out = out + bias[n]]
      [gated: up = (f32(acc_up) * x_scale[m]) * w_scale[N + n];  out = silu(out) * up, in float64]
      [out = out + residual];  [mix: out = (f32(round(out)) * rs) + (original * is)];  round to out_dtype.
    """
    rows, K = weight.shape
    N = rows // 2 if gated else rows
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    acc = int8_accumulate(x2, weight)
    xs = np.asarray(x_scale, dtype=F32).reshape(-1)[:, None]
    ws = np.asarray(weight_scale, dtype=F32).reshape(-1)
    out = (acc[:, :N].astype(F32) * xs) * ws[None, :N]
    if bias is not None:
        out = out + np.asarray(bias).astype(F32)[None, :]
    if gated:
        up = (acc[:, N:].astype(F32) * xs) * ws[None, N:]
        out = silu_product(out, up)
    if residual is not None:
        out = out + np.asarray(residual).reshape(M, N).astype(F32)
    if original is not None:
        stream = round_to(out, out_dtype).astype(F32)
        out = mix(stream, np.asarray(original).reshape(M, N), residual_scale, input_scale, F32)
    return round_to(out, out_dtype).reshape(*x.shape[:-1], N)


def linear(x, weight, bias=None, residual=None, gated=False, accumulate_fp32=False, original=None, residual_scale=None,
           input_scale=None) -> np.ndarray:
    """model/fused_blocks.py:229-318, w in_features x out_features; sums in float64 (the kernel sums fp16 products in
    f32 on MFMA, the reference in fp16: neither order is bitwise reproducible, so this is the tolerance reference).
    fp16 out, or f32 with accumulate_fp32."""
    K, width = weight.shape
    N = width // 2 if gated else width
    x2 = np.asarray(x).reshape(-1, K).astype(np.float64)
    acc = x2 @ np.asarray(weight).astype(np.float64)
    out = acc[:, :N]
    if bias is not None:
        out = out + np.asarray(bias).astype(np.float64)[None, :]
    if gated:
        out = out / (1.0 + np.exp(-out)) * acc[:, N:]
    if residual is not None:
        out = out + np.asarray(residual).reshape(-1, N).astype(np.float64)
    dtype = F32 if accumulate_fp32 else F16
    if original is not None:
        stream = out.astype(dtype).astype(np.float64)
        rs = float(np.asarray(residual_scale, dtype=np.float32).reshape(-1)[0])
        is_ = float(np.asarray(input_scale, dtype=np.float32).reshape(-1)[0])
        out = rs * stream + is_ * np.asarray(original).reshape(-1, N).astype(np.float64)
    return out.astype(dtype).reshape(*np.asarray(x).shape[:-1], N)


NUM_SQUARES = 64


def template_attention(projected, templates, q_gain, k_gain, heads, kv_heads, dq, dv, templates_count, eps) -> np.ndarray:
    """model/fused_blocks.py:54-97 and :104-171: per-head RMSNorm of q (rounded to fp16) and k (rounded to fp16),
    s = q k^T / sqrt(dq), plus on square x square the template bias sum_t c[b,i,h,t] templates[t,i,j] rounded to
    fp16; softmax over the T keys with the probabilities rounded to fp16 before P V, divided by the f32 row sum.
    Float64 sums; returns f32 [B, T, heads * dv] (the kernel rounds to fp16)."""
    projected = np.asarray(projected)
    B, T, _ = projected.shape
    p = projected.astype(np.float64)
    splits = np.cumsum([heads * dq, kv_heads * dq, kv_heads * dv])
    q, k, v, c = np.split(p, splits, axis=-1)
    per_kv = heads // kv_heads

    def head_norm(values, gain, count):
        values = values.reshape(B, T, count, dq)
        inverse = 1.0 / np.sqrt((values * values).mean(-1, keepdims=True) + eps)
        return (values * inverse * np.asarray(gain).astype(np.float64)).astype(F16).astype(np.float64)

    qn = head_norm(q, q_gain, heads)                                     # B T H dq
    kn = np.repeat(head_norm(k, k_gain, kv_heads), per_kv, axis=2)       # B T H dq
    vh = np.repeat(v.reshape(B, T, kv_heads, dv), per_kv, axis=2)        # B T H dv
    scores = np.einsum("bihd,bjhd->bhij", qn, kn) / math.sqrt(dq)
    coefficients = c[:, :NUM_SQUARES].reshape(B, NUM_SQUARES, heads, templates_count)
    bias = np.einsum("biht,tij->bhij", coefficients, np.asarray(templates).astype(np.float64)[:templates_count])
    scores[:, :, :NUM_SQUARES, :NUM_SQUARES] += bias.astype(F16).astype(np.float64)
    scores -= scores.max(-1, keepdims=True)
    probabilities = np.exp(scores)
    total = probabilities.sum(-1, keepdims=True)
    weighted = np.einsum("bhij,bjhd->bhid", probabilities.astype(F16).astype(np.float64), vh) / total
    return weighted.transpose(0, 2, 1, 3).reshape(B, T, heads * dv).astype(F32)


def int8_block_forward(x, templates, original, block: dict, input_mixed: bool, next_scales=None, rounded_attention=True):
    """model/int8_blocks.py:274-288, one Int8Block: returns the block's fp16 output (the next block's mixed input when
    next_scales is given). ``block`` holds the Int8Block's buffers as numpy arrays under their attribute names."""
    eps = block["eps"]
    if input_mixed:
        normed, scale = norm_quant(x, block["ln1"], eps)
    else:
        x, normed, scale = mix_norm_quant(x, original, block["residual_scale"], block["input_scale"], block["ln1"], eps)
    projected = int8_linear(normed, scale, block["projection"], block["projection_scale"], block["projection_bias"])
    attended = template_attention(projected, templates, block["q_gain"], block["k_gain"], block["heads"], block["kv_heads"],
                                  block["dq"], block["dv"], block["templates_count"], eps)
    if rounded_attention:
        attended = attended.astype(F16)
    x = linear(attended, block["combine_heads"], block["combine_heads_bias"], residual=x)
    normed, scale = norm_quant(x, block["ln2"], eps)
    hidden = int8_linear(normed, scale, block["gate_up"], block["gate_up_scale"], gated=True)
    rotated, scale = rotate_quant(hidden, block["down"].shape[1])
    if next_scales is None:
        return int8_linear(rotated, scale, block["down"], block["down_scale"], residual=x)
    return int8_linear(rotated, scale, block["down"], block["down_scale"], residual=x, original=original,
                       residual_scale=next_scales[0], input_scale=next_scales[1])
