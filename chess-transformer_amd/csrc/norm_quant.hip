// RMSNorm + per-row int8 quantisation, optionally mixing in the block's input first.
// Computes what model/int8_blocks.py:156-175 (norm_quant_kernel) does, in a declared op order:
//   [mixed = f16((x * rs) + (original * is))]
//   y = (x * (1 / sqrt(tree_sum(x * x) / D + eps))) * gain
//   absmax = max(max |y|, 1e-20);  q = rint(y * (127 / absmax));  scale = absmax / 127
// One wavefront per row; a lane holds C = next_pow2(D) / 64 contiguous elements (at least 1),
// sums its squares as a pairwise tree and the wavefront adds the lanes' sums by xor butterflies,
// which is the balanced tree over the zero-padded row. Bandwidth-bound: 16-byte loads and stores.
#include "chess_common.h"

namespace {

constexpr int ROWS_PER_BLOCK = 4;

template <int BYTES> struct Bytes;
template <> struct Bytes<1> { typedef uint8_t type; };
template <> struct Bytes<2> { typedef uint16_t type; };
template <> struct Bytes<4> { typedef uint32_t type; };
template <> struct Bytes<8> { typedef uint2 type; };
template <> struct Bytes<16> { typedef uint4 type; };

template <int BYTES> DEVICE void copy_bytes(void* to, const void* from) {
    if constexpr (BYTES <= 16) {
        *reinterpret_cast<typename Bytes<BYTES>::type*>(to) = *reinterpret_cast<const typename Bytes<BYTES>::type*>(from);
    } else {
#pragma unroll
        for (int i = 0; i < BYTES / 16; i++) reinterpret_cast<uint4*>(to)[i] = reinterpret_cast<const uint4*>(from)[i];
    }
}

// C halves from row[col..col+C): one vector load when the row length is a multiple of C, else element by element.
template <int C> DEVICE void load_halves(const half_t* row, int col, int D, bool vector, float (&out)[C]) {
    half_t raw[C];
    if (vector) {
        if (col < D) {
            copy_bytes<2 * C>(raw, row + col);
        } else {
#pragma unroll
            for (int i = 0; i < C; i++) raw[i] = (half_t)0.0f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < C; i++) raw[i] = col + i < D ? row[col + i] : (half_t)0.0f;
    }
#pragma unroll
    for (int i = 0; i < C; i++) out[i] = (float)raw[i];
}

template <int C>
__global__ __launch_bounds__(64 * ROWS_PER_BLOCK) void norm_quant_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ original, const half_t* __restrict__ residual_scale,
    const half_t* __restrict__ input_scale, const half_t* __restrict__ gain, half_t* __restrict__ mixed,
    int8_t* __restrict__ q, float* __restrict__ scale, int M, int D, float eps, int mix)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= M) return;  // the whole wavefront leaves together
    const bool vector = D % C == 0;
    const int col = lane * C;
    const size_t base = (size_t)row * D;

    float v[C];
    load_halves<C>(x + base, col, D, vector, v);
    if (mix) {
        float o[C];
        load_halves<C>(original + base, col, D, vector, o);
        const float rs = (float)residual_scale[0], is = (float)input_scale[0];
        half_t m[C];
#pragma unroll
        for (int i = 0; i < C; i++) {
            m[i] = (half_t)((v[i] * rs) + (o[i] * is));
            v[i] = (float)m[i];
        }
        if (vector) {
            if (col < D) copy_bytes<2 * C>(mixed + base + col, m);
        } else {
#pragma unroll
            for (int i = 0; i < C; i++)
                if (col + i < D) mixed[base + col + i] = m[i];
        }
    }

    // the lane's squares as a pairwise tree, then the wavefront's butterflies
    float squares[C];
#pragma unroll
    for (int i = 0; i < C; i++) squares[i] = v[i] * v[i];
#pragma unroll
    for (int width = C; width > 1; width >>= 1)
#pragma unroll
        for (int i = 0; i < width / 2; i++) squares[i] = squares[2 * i] + squares[2 * i + 1];
    const float total = wave_sum(squares[0]);
    const float inverse = 1.0f / __builtin_sqrtf(total / (float)D + eps);

    float y[C];
    float largest = 0.0f;
#pragma unroll
    for (int i = 0; i < C; i++) {
        const float g = col + i < D ? (float)gain[col + i] : 0.0f;
        y[i] = (v[i] * inverse) * g;
        largest = fmaxf(largest, fabsf(y[i]));
    }
    const float absmax = fmaxf(wave_max(largest), 1e-20f);
    const float inverse_step = 127.0f / absmax;
    int8_t out[C];
#pragma unroll
    for (int i = 0; i < C; i++) out[i] = (int8_t)(int)__builtin_rintf(y[i] * inverse_step);
    if (vector) {
        if (col < D) copy_bytes<C>(q + base + col, out);
    } else {
#pragma unroll
        for (int i = 0; i < C; i++)
            if (col + i < D) q[base + col + i] = out[i];
    }
    if (lane == 0) scale[row] = absmax / 127.0f;
}

template <int C>
int launch(const void* x, const void* original, const void* residual_scale, const void* input_scale, const void* gain, void* mixed,
           void* q, void* scale, int M, int D, float eps, hipStream_t stream)
{
    const dim3 grid((M + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK), block(64 * ROWS_PER_BLOCK);
    hipLaunchKernelGGL(norm_quant_kernel<C>, grid, block, 0, stream, (const half_t*)x, (const half_t*)original,
                       (const half_t*)residual_scale, (const half_t*)input_scale, (const half_t*)gain, (half_t*)mixed, (int8_t*)q,
                       (float*)scale, M, D, eps, original != nullptr ? 1 : 0);
    return launch_status();
}

}  // namespace

extern "C" int chess_norm_quant(const void* x, const void* original, const void* residual_scale, const void* input_scale,
                                const void* gain, void* mixed, void* q, void* scale, int M, int D, float eps, void* stream)
{
    if (M < 0 || D <= 0) return chess_fail(CHESS_INVALID_SHAPE, "norm_quant: rows %d and width %d", M, D);
    if (D > 64 * 32) return chess_fail(CHESS_UNSUPPORTED, "norm_quant takes rows of at most 2048, not %d", D);
    if (!x || !gain || !q || !scale) return chess_fail(CHESS_INVALID_SHAPE, "norm_quant: a required pointer is null");
    if (original && (!residual_scale || !input_scale || !mixed))
        return chess_fail(CHESS_INVALID_SHAPE, "mix_norm_quant needs the scales and the mixed output");
    if (!aligned16(x) || !aligned16(q) || (original && (!aligned16(original) || !aligned16(mixed))))
        return chess_fail(CHESS_MISALIGNED, "norm_quant's vector loads need 16-byte aligned rows");
    if (M == 0) return CHESS_OK;
    int padded = 64;
    while (padded < D) padded <<= 1;
    hipStream_t s = (hipStream_t)stream;
    switch (padded / 64) {
        case 1: return launch<1>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
        case 2: return launch<2>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
        case 4: return launch<4>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
        case 8: return launch<8>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
        case 16: return launch<16>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
        default: return launch<32>(x, original, residual_scale, input_scale, gain, mixed, q, scale, M, D, eps, s);
    }
}
