// The policy head's move logits of B positions, from the final norm's rows, one workgroup a position.
// Computes what model/fused_blocks.py:863-872 (the heads without fused ends) computes after its `a` matmul:
//   narrow[t][c] = x[t] . W[c] + w_bias[c]                          c < NN: s, the promotion logits, board_down's
//   logits[i][j] = (a[i] + a_bias) . x[j] + narrow[i][0]             i, j < 64, the squares
//   out[m] = logits[from m][to m] (+ narrow[to'][column'] for a promotion move)
// and writes board_down's inputs narrow[t][down_first..NN) for the value head. x is the stream [B, T, D] fp16 (exact
// in f32), a [B, T, D] f32 (rows 0..63 read), a_bias [D], W [NN, D] and w_bias [NN] f32. The reference takes these
// products in f32 (torch's F.linear and bmm); here they are f32 MFMAs (v_mfma_f32_32x32x2_f32: exact products,
// f32 sums), so the results agree with it to f32 rounding, not to the bit.
//
// Four wavefronts: each takes a 32 x 32 quadrant of the logits, and wavefronts 0-2 a block of 32 token rows of the
// narrow products (all NN <= 32 columns). A step covers 8 of D: lane l (row l % 32, half h = l / 32) loads 4
// consecutive values k0 + 4h .. + 3 of its row of each operand and feeds them to 4 MFMAs, value m to MFMA m, so
// that in MFMA m both operands' k-halves stand for k0 + m and k0 + 4 + m; eight steps' loads go out together. The
// quadrants and the narrow rows meet in LDS for the gather of the 1,968 moves.
#include "chess_common.h"

namespace {

constexpr int SQUARES = 64;
constexpr int MAX_NARROW = 32;
constexpr int MAX_TOKENS = 96;                 // three blocks of 32 token rows
constexpr int LOGIT_STRIDE = SQUARES + 1;
constexpr int NARROW_STRIDE = MAX_NARROW + 1;
constexpr int THREADS = 256;

typedef float v16f __attribute__((ext_vector_type(16)));

DEVICE v16f mfma_f32(float a, float b, v16f c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }

// the 32 x 32 block sum_k A[row0 + i][k] * X[col0 + j][k] over k < D: A's rows f32 (a_bias added when BIAS), X's fp16;
// rows past a_rows and columns past x_rows read the last one (never kept). Lane l holds, in register 4q + r,
// the sum for A row 8q + 4(l / 32) + r and X row l % 32. D is a multiple of 64: eight steps a turn, their loads
// issued before their MFMAs, so that a turn's loads are in flight together.
template <bool BIAS>
DEVICE v16f block_products(const float* A, int a_rows, const float* a_bias, const half_t* X, int x_rows, int D, int lane) {
    constexpr int TURN = 8;   // steps of 8 a turn
    const int r32 = lane & 31, h = lane >> 5;
    const float* a_row = A + (size_t)min(r32, a_rows - 1) * D + 4 * h;
    const half_t* x_row = X + (size_t)min(r32, x_rows - 1) * D + 4 * h;
    v16f acc = {};
    for (int turn = 0; turn < D; turn += 8 * TURN) {
        float4 av[TURN];
        v4h xv[TURN];
#pragma unroll
        for (int s = 0; s < TURN; s++) {
            av[s] = *reinterpret_cast<const float4*>(a_row + turn + 8 * s);
            xv[s] = *reinterpret_cast<const v4h*>(x_row + turn + 8 * s);
        }
#pragma unroll
        for (int s = 0; s < TURN; s++) {
            float4 a4 = av[s];
            if constexpr (BIAS) {
                const float4 bias = *reinterpret_cast<const float4*>(a_bias + turn + 8 * s + 4 * h);
                a4 = float4{a4.x + bias.x, a4.y + bias.y, a4.z + bias.z, a4.w + bias.w};
            }
            acc = mfma_f32(a4.x, (float)xv[s][0], acc);
            acc = mfma_f32(a4.y, (float)xv[s][1], acc);
            acc = mfma_f32(a4.z, (float)xv[s][2], acc);
            acc = mfma_f32(a4.w, (float)xv[s][3], acc);
        }
    }
    return acc;
}

__global__ __launch_bounds__(THREADS) void move_logits_kernel(
    const half_t* __restrict__ x, const float* __restrict__ a, const float* __restrict__ a_bias, const float* __restrict__ w,
    const float* __restrict__ w_bias, const int* __restrict__ cells, const int* __restrict__ promotions, float* __restrict__ out,
    float* __restrict__ down, int T, int D, int NN, int down_first, int moves)
{
    __shared__ float logits[SQUARES * LOGIT_STRIDE];
    __shared__ float narrow[MAX_TOKENS * NARROW_STRIDE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t b = blockIdx.x;
    const half_t* xb = x + b * T * D;
    const int r32 = lane & 31, h = lane >> 5;

    // the wavefront's quadrant of a . x^T: rows i0.. of a (the from side), columns j0.. of x (the to side)
    const int i0 = (wave >> 1) * 32, j0 = (wave & 1) * 32;
    const v16f quadrant = block_products<true>(a + (b * T + i0) * D, 32, a_bias, xb + (size_t)j0 * D, 32, D, lane);

    // narrow[t][c] for the wavefront's 32 token rows: W's rows (columns c) as the first operand, x's as the second
    if (wave < 3) {
        const int t0 = wave * 32;
        if (t0 < T) {
            const v16f products = block_products<false>(w, NN, nullptr, xb + (size_t)t0 * D, T - t0, D, lane);
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int c = 8 * q + 4 * h + r, t = t0 + r32;
                    if (c < NN && t < T) narrow[t * NARROW_STRIDE + c] = products[4 * q + r] + w_bias[c];
                }
        }
    }
    __syncthreads();

    // logits = the quadrant + s[i] (the from square's narrow column 0)
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = i0 + 8 * q + 4 * h + r, j = j0 + r32;
            logits[i * LOGIT_STRIDE + j] = quadrant[4 * q + r] + narrow[i * NARROW_STRIDE];
        }
    __syncthreads();

    // the moves: cells[m] = from * 64 + to; promotions[m] = to' * 32 + column of its promotion logit, or -1 (the places
    // are masked into the tiles, so that no table entry reads outside them)
    float* out_b = out + b * moves;
    for (int m = tid; m < moves; m += THREADS) {
        const int cell = cells[m], promotion = promotions[m];
        float value = logits[((cell >> 6) & 63) * LOGIT_STRIDE + (cell & 63)];
        if (promotion >= 0) value = value + narrow[((promotion >> 5) & 63) * NARROW_STRIDE + (promotion & 31)];
        out_b[m] = value;
    }
    const int width = NN - down_first;
    float* down_b = down + b * T * width;
    for (int e = tid; e < T * width; e += THREADS) down_b[e] = narrow[(e / width) * NARROW_STRIDE + down_first + e % width];
}

}  // namespace

extern "C" int chess_move_logits(const void* x, const void* a, const void* a_bias, const void* w, const void* w_bias, const void* cells,
                                 const void* promotions, void* out, void* down, int B, int T, int D, int NN, int down_first, int moves,
                                 void* stream)
{
    if (B < 0 || T < SQUARES || T > MAX_TOKENS || D <= 0 || D % 64 != 0)
        return chess_fail(CHESS_UNSUPPORTED, "move_logits takes %d to %d tokens of a width that is a multiple of 64, not %d x %d", SQUARES, MAX_TOKENS,
                          T, D);
    if (NN <= 0 || NN > MAX_NARROW || down_first < 1 || down_first > NN || moves <= 0)
        return chess_fail(CHESS_INVALID_SHAPE, "move_logits: %d narrow columns (at most %d), board_down from %d, %d moves", NN, MAX_NARROW,
                          down_first, moves);
    if (!x || !a || !a_bias || !w || !w_bias || !cells || !promotions || !out || !down)
        return chess_fail(CHESS_INVALID_SHAPE, "move_logits: a required pointer is null");
    if (!aligned16(x) || !aligned16(a) || !aligned16(a_bias) || !aligned16(w))
        return chess_fail(CHESS_MISALIGNED, "move_logits reads x, a, a_bias and W 8 and 16 bytes a lane");
    if (B == 0) return CHESS_OK;
    hipLaunchKernelGGL(move_logits_kernel, dim3(B), dim3(THREADS), 0, (hipStream_t)stream, (const half_t*)x, (const float*)a,
                       (const float*)a_bias, (const float*)w, (const float*)w_bias, (const int*)cells, (const int*)promotions, (float*)out,
                       (float*)down, T, D, NN, down_first, moves);
    return launch_status();
}
