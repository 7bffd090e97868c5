// RMSNorm + per-row int8 quantisation, optionally mixing in the block's input first.
// Computes what model/int8_blocks.py:156-175 (norm_quant_kernel) does, in a declared op order:
//   [mixed = f16((x * rs) + (original * is))]
//   y = (x * (1 / sqrt(tree_sum(x * x) / D + eps))) * gain
//   absmax = max(max |y|, 1e-20);  q = rint(y * (127 / absmax));  scale = absmax / 127
// Without the quantisation (QUANT false) the same kernel is the fp16 blocks' RMSNorm: out = f16(y), after the same
// optional mix (model/fused_blocks.py:346-348 and :351, and the final norm at :863).
// A wavefront takes R rows, one at a time, after loading all of them; a lane holds C = next_pow2(D) / 64
// contiguous elements of a row (at least 1), sums its squares as a pairwise tree and the wavefront adds
// the lanes' sums as a balanced tree of adjacent lanes, which is the balanced tree over the zero-padded row.
// Bandwidth-bound: 16-byte loads and stores, R rows of loads in flight a wavefront.
#include "chess_common.h"

namespace {

constexpr int WAVES = 4;   // wavefronts a workgroup

// naturally aligned vector types of 1 to 16 bytes: a copy of BYTES is one load or store of that width
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
template <int BYTES> struct Bytes;
template <> struct Bytes<1> { typedef uint8_t type; };
template <> struct Bytes<2> { typedef uint16_t type; };
template <> struct Bytes<4> { typedef uint32_t type; };
template <> struct Bytes<8> { typedef v2u type; };
template <> struct Bytes<16> { typedef v4u type; };

template <int BYTES> DEVICE void copy_bytes(void* to, const void* from) {
    if constexpr (BYTES <= 16) {
        *reinterpret_cast<typename Bytes<BYTES>::type*>(to) = *reinterpret_cast<const typename Bytes<BYTES>::type*>(from);
    } else {
#pragma unroll
        for (int i = 0; i < BYTES / 16; i++) reinterpret_cast<v4u*>(to)[i] = reinterpret_cast<const v4u*>(from)[i];
    }
}

// C halves from row[col..col+C) (the caller zeroes those past D): one vector load when the row length is a multiple
// of C, from a place clamped into the row, so that no branch holds the load back and the loads of several rows stay in
// flight together; else element by element.
template <int C, bool VECTOR> DEVICE void load_raw(const half_t* row, int col, int D, half_t (&raw)[C]) {
    if constexpr (VECTOR) {
        copy_bytes<2 * C>(raw, row + min(col, D - C));
    } else {
#pragma unroll
        for (int i = 0; i < C; i++) raw[i] = row[min(col + i, D - 1)];
    }
}

// FULL: the row is exactly 64 lanes of C (D == 64 C), so no element is past the row and nothing is masked
template <int C, bool FULL> DEVICE void widen(const half_t (&raw)[C], int col, int D, float (&out)[C]) {
#pragma unroll
    for (int i = 0; i < C; i++) out[i] = FULL || col + i < D ? (float)raw[i] : 0.0f;
}

template <int C, int R, bool VECTOR, bool QUANT, bool FULL = false>
__global__ __launch_bounds__(64 * WAVES) void norm_quant_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ original, const half_t* __restrict__ residual_scale,
    const half_t* __restrict__ input_scale, const half_t* __restrict__ gain, half_t* __restrict__ mixed,
    int8_t* __restrict__ q, float* __restrict__ scale, half_t* __restrict__ normed, int M, int D, float eps, int mix)
{
    const int lane = threadIdx.x & 63;
    const int first = (blockIdx.x * WAVES + (threadIdx.x >> 6)) * R;
    if (first >= M) return;  // the whole wavefront leaves together
    constexpr bool vector = VECTOR;
    const int col = lane * C;

    // the wavefront's R rows (and inputs) are loaded before any is used, so that R rows of loads are in flight
    half_t raw_x[R][C], raw_o[R][C];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(first + r, M - 1);
        load_raw<C, VECTOR>(x + (size_t)row * D, col, D, raw_x[r]);
        if (mix) load_raw<C, VECTOR>(original + (size_t)row * D, col, D, raw_o[r]);
    }
    // the gain: one vector load when the row is full (the launch checks its alignment), else element by element
    half_t raw_g[C];
    if constexpr (FULL) copy_bytes<2 * C>(raw_g, gain + col);
    else load_raw<C, false>(gain, col, D, raw_g);
    float g[C];
    widen<C, FULL>(raw_g, col, D, g);
    float rs = 0.0f, is = 0.0f;
    if (mix) {
        rs = (float)residual_scale[0];
        is = (float)input_scale[0];
    }

#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = first + r;
        if (row >= M) break;
        const size_t base = (size_t)row * D;
        float v[C];
        widen<C, FULL>(raw_x[r], col, D, v);
        if (mix) {
            float o[C];
            widen<C, FULL>(raw_o[r], col, D, o);
            half_t m[C];
#pragma unroll
            for (int i = 0; i < C; i++) {
                m[i] = (half_t)((v[i] * rs) + (o[i] * is));
                v[i] = (float)m[i];
            }
            if (vector) {
                if (FULL || col < D) copy_bytes<2 * C>(mixed + base + col, m);
            } else {
#pragma unroll
                for (int i = 0; i < C; i++)
                    if (col + i < D) mixed[base + col + i] = m[i];
            }
        }

        if constexpr (QUANT) {
            int8_t out[C];
            const float absmax = norm_quant_row<C>(v, g, D, eps, out);
            if (vector) {
                if (FULL || col < D) copy_bytes<C>(q + base + col, out);
            } else {
#pragma unroll
                for (int i = 0; i < C; i++)
                    if (col + i < D) q[base + col + i] = out[i];
            }
            if (lane == 0) scale[row] = absmax / 127.0f;
        } else {
            const float inverse = rms_inverse<C>(v, D, eps);
            half_t out[C];
#pragma unroll
            for (int i = 0; i < C; i++) {
                float y = (v[i] * inverse) * g[i];
                asm volatile("" : "+v"(y));   // the f32 product rounds to fp16 (one rounding of y, not a mixed multiply)
                out[i] = (half_t)y;
            }
            if (vector) {
                if (FULL || col < D) copy_bytes<2 * C>(normed + base + col, out);
            } else {
#pragma unroll
                for (int i = 0; i < C; i++)
                    if (col + i < D) normed[base + col + i] = out[i];
            }
        }
    }
}

template <int C, bool QUANT>
int launch(const void* x, const void* original, const void* residual_scale, const void* input_scale, const void* gain, void* mixed,
           void* q, void* scale, void* normed, int M, int D, float eps, hipStream_t stream)
{
    // rows a wavefront: two once the launch fills the chip (at 71,680 rows of 512 one row takes 41.5 us, two 29.1, four
    // 30.0, eight 31.2 on an MI355X), one row a wavefront while it does not
    constexpr int WIDE = 2;
    const bool wide = M >= 32768;
    const int rows_per_block = WAVES * (wide ? WIDE : 1);
    const dim3 grid((M + rows_per_block - 1) / rows_per_block), block(64 * WAVES);
    // a full row (D == 64 C) with a 16-byte aligned gain takes no masks and loads the gain as vectors (at 71,680 rows
    // of 512 on an MI355X: 28.8 us, from 32.5 us with the masks and the gain's element loads)
    const bool full = D == 64 * C && aligned16(gain);
    auto kernel = wide ? (full ? norm_quant_kernel<C, WIDE, true, QUANT, true>
                               : D % C == 0 ? norm_quant_kernel<C, WIDE, true, QUANT> : norm_quant_kernel<C, WIDE, false, QUANT>)
                       : (full ? norm_quant_kernel<C, 1, true, QUANT, true>
                               : D % C == 0 ? norm_quant_kernel<C, 1, true, QUANT> : norm_quant_kernel<C, 1, false, QUANT>);
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, (const half_t*)x, (const half_t*)original, (const half_t*)residual_scale,
                       (const half_t*)input_scale, (const half_t*)gain, (half_t*)mixed, (int8_t*)q, (float*)scale, (half_t*)normed, M, D,
                       eps, original != nullptr ? 1 : 0);
    return launch_status();
}

template <bool QUANT>
int by_width(const void* x, const void* original, const void* residual_scale, const void* input_scale, const void* gain, void* mixed, void* q,
             void* scale, void* normed, int M, int D, float eps, hipStream_t s)
{
    int padded = 64;
    while (padded < D) padded <<= 1;
    switch (padded / 64) {
        case 1: return launch<1, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
        case 2: return launch<2, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
        case 4: return launch<4, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
        case 8: return launch<8, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
        case 16: return launch<16, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
        default: return launch<32, QUANT>(x, original, residual_scale, input_scale, gain, mixed, q, scale, normed, M, D, eps, s);
    }
}

int check_rows(const void* x, const void* original, const void* residual_scale, const void* input_scale, const void* gain, void* mixed,
               int M, int D, const char* what)
{
    if (M < 0 || D <= 0) return chess_fail(CHESS_INVALID_SHAPE, "%s: rows %d and width %d", what, M, D);
    if (D > 64 * 32) return chess_fail(CHESS_UNSUPPORTED, "%s takes rows of at most 2048, not %d", what, D);
    if (!x || !gain) return chess_fail(CHESS_INVALID_SHAPE, "%s: a required pointer is null", what);
    if (original && (!residual_scale || !input_scale || !mixed))
        return chess_fail(CHESS_INVALID_SHAPE, "%s's input mix needs the scales and the mixed output", what);
    if (!aligned16(x) || (original && (!aligned16(original) || !aligned16(mixed))))
        return chess_fail(CHESS_MISALIGNED, "%s's vector loads need 16-byte aligned rows", what);
    return CHESS_OK;
}

}  // namespace

extern "C" int chess_norm_quant(const void* x, const void* original, const void* residual_scale, const void* input_scale,
                                const void* gain, void* mixed, void* q, void* scale, int M, int D, float eps, void* stream)
{
    if (int status = check_rows(x, original, residual_scale, input_scale, gain, mixed, M, D, "norm_quant")) return status;
    if (!q || !scale) return chess_fail(CHESS_INVALID_SHAPE, "norm_quant: a required pointer is null");
    if (!aligned16(q)) return chess_fail(CHESS_MISALIGNED, "norm_quant's vector loads need 16-byte aligned rows");
    if (M == 0) return CHESS_OK;
    return by_width<true>(x, original, residual_scale, input_scale, gain, mixed, q, scale, nullptr, M, D, eps, (hipStream_t)stream);
}

extern "C" int chess_rms_norm(const void* x, const void* original, const void* residual_scale, const void* input_scale, const void* gain,
                              void* mixed, void* out, int M, int D, float eps, void* stream)
{
    if (int status = check_rows(x, original, residual_scale, input_scale, gain, mixed, M, D, "rms_norm")) return status;
    if (!out) return chess_fail(CHESS_INVALID_SHAPE, "rms_norm: a required pointer is null");
    if (!aligned16(out)) return chess_fail(CHESS_MISALIGNED, "rms_norm's vector loads need 16-byte aligned rows");
    if (M == 0) return CHESS_OK;
    return by_width<false>(x, original, residual_scale, input_scale, gain, mixed, nullptr, nullptr, out, M, D, eps, (hipStream_t)stream);
}
