// W8A8 GEMM on CDNA4 int8 MFMA with the int8_linear epilogues.
// Computes what model/int8_blocks.py:66-144 (int8_linear_kernel) and model/int8_cuda.py:34-183
// (small_int8) compute: out[M, N] = epilogue(x[M, K] @ w[N, K]^T), x and w int8, exact int32 sums.
// Epilogue op order (f32, one IEEE op per step, no fma):
//   v = f32(acc) * x_scale[m];  out = v * w_scale[n]
//   [BIAS]      out = out + bias[n]
//   [GATED]     up = (f32(acc_up) * x_scale[m]) * w_scale[N + n];  out = silu(out) * up
//   [RESIDUAL]  out = out + residual[m, n]
//   [MIX]       out = (f32(round(out)) * residual_scale) + (original[m, n] * input_scale)
//   round to fp16 / bf16 (or, for the accumulator entry point, the raw int32 sums).
// The int32 sums are exact in any order, and every tile shape runs the same epilogue, so the tile
// chosen for a shape never changes a bit.
//
// Layout: x row-major [M, K], w row-major [N(x2 gated), K] (the gate's rows, then up's), K % 64 == 0.
// A workgroup of 4 wavefronts takes a BM x BN tile; each wavefront a (BM/2) x (BN/2) quarter as
// 16x16 fragments of v_mfma_i32_16x16x64_i8. K advances 64 at a time through double-buffered LDS,
// the next step's 16-byte global loads in flight while the current step's MFMAs run. An MFMA
// operand lane holds 16 consecutive bytes of one row, so both operands are read from LDS as plain
// 16-byte rows; which k a byte position stands for is the same for both operands, so the sums
// are the dot products whatever the hardware's k order.
#include "chess_common.h"

#include <type_traits>

namespace {

constexpr int BK = 64;
constexpr int THREADS = 256;

enum { EPI_BIAS = 1, EPI_RESIDUAL = 2, EPI_MIX = 4 };

struct Epilogue {
    const float* x_scale;
    const float* w_scale;
    const half_t* bias;
    const half_t* residual;
    const half_t* original;
    const half_t* residual_scale;
    const half_t* input_scale;
    int flags;
};

template <int BM, int BN, int NB, typename OutT>
__global__ __launch_bounds__(THREADS) void int8_gemm_kernel(
    const int8_t* __restrict__ x, const int8_t* __restrict__ w, OutT* __restrict__ out, Epilogue e, int M, int N, int K)
{
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int A_CHUNKS = BM * BK / 16 / THREADS;
    constexpr int B_CHUNKS = NB * BN * BK / 16 / THREADS;
    static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for the loaders");
    __shared__ __align__(16) int8_t lds_a[2][BM * BK];
    __shared__ __align__(16) int8_t lds_b[2][NB * BN * BK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const int tile = xcd_local_tile(blockIdx.x, tiles_m * tiles_n);
    constexpr int GROUP_M = 8;
    const int in_group = GROUP_M * tiles_n;
    const int first_m = tile / in_group * GROUP_M;
    const int group_rows = min(tiles_m - first_m, GROUP_M);
    const int m0 = (first_m + tile % in_group % group_rows) * BM;
    const int n0 = (tile % in_group / group_rows) * BN;

    // rows past M read row M - 1 and columns past N read column N - 1: their sums are never stored
    const int8_t* a_src[A_CHUNKS];
    int a_dst[A_CHUNKS];
#pragma unroll
    for (int c = 0; c < A_CHUNKS; c++) {
        const int idx = tid + c * THREADS, r = idx >> 2, part = idx & 3;
        a_src[c] = x + (size_t)min(m0 + r, M - 1) * K + part * 16;
        a_dst[c] = r * BK + part * 16;
    }
    const int8_t* b_src[B_CHUNKS];
    int b_dst[B_CHUNKS];
#pragma unroll
    for (int c = 0; c < B_CHUNKS; c++) {
        const int idx = tid + c * THREADS, r = idx >> 2, part = idx & 3;
        const int group = r / BN, col = min(n0 + r % BN, N - 1);
        b_src[c] = w + ((size_t)group * N + col) * K + part * 16;
        b_dst[c] = r * BK + part * 16;
    }

    uint4 a_reg[A_CHUNKS], b_reg[B_CHUNKS];

    v4i acc[NB][FM][FN];
#pragma unroll
    for (int g = 0; g < NB; g++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[g][i][j] = v4i{0, 0, 0, 0};

    const int steps = K / BK;
    const int row_in = lane & 15, part_in = (lane >> 4) * 16;
    {
        const int k0 = 0;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) a_reg[c] = *reinterpret_cast<const uint4*>(a_src[c] + k0);
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++) b_reg[c] = *reinterpret_cast<const uint4*>(b_src[c] + k0);
    }
    {
        const int buffer = 0;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_a[buffer][a_dst[c]]) = a_reg[c];
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_b[buffer][b_dst[c]]) = b_reg[c];
    }
    __syncthreads();
    for (int step = 0; step < steps; step++) {
        const int buffer = step & 1;
        {
            // the last step loads its own tile again: no branch, so the prefetch stays in registers
            const int k0 = min(step + 1, steps - 1) * BK;
#pragma unroll
            for (int c = 0; c < A_CHUNKS; c++) a_reg[c] = *reinterpret_cast<const uint4*>(a_src[c] + k0);
#pragma unroll
            for (int c = 0; c < B_CHUNKS; c++) b_reg[c] = *reinterpret_cast<const uint4*>(b_src[c] + k0);
        }
        v4i af[FM];
#pragma unroll
        for (int i = 0; i < FM; i++)
            af[i] = *reinterpret_cast<const v4i*>(&lds_a[buffer][(wm * WM + i * 16 + row_in) * BK + part_in]);
#pragma unroll
        for (int g = 0; g < NB; g++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const v4i bf = *reinterpret_cast<const v4i*>(&lds_b[buffer][(g * BN + wn * WN + j * 16 + row_in) * BK + part_in]);
#pragma unroll
                for (int i = 0; i < FM; i++) acc[g][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf, acc[g][i][j], 0, 0, 0);
            }
        {
            const int next = buffer ^ 1;
#pragma unroll
            for (int c = 0; c < A_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_a[next][a_dst[c]]) = a_reg[c];
#pragma unroll
            for (int c = 0; c < B_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_b[next][b_dst[c]]) = b_reg[c];
        }
        __syncthreads();
    }

    // a fragment's lane holds column lane % 16 of rows 4 * (lane / 16) + r
    const int col_in = lane & 15, row_base = (lane >> 4) * 4;
    float rs = 0.0f, is = 0.0f;
    if (e.flags & EPI_MIX) {
        rs = (float)e.residual_scale[0];
        is = (float)e.input_scale[0];
    }
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int n = n0 + wn * WN + j * 16 + col_in;
        if (n >= N) continue;
        float ws = 0.0f, ws_up = 0.0f, b = 0.0f;
        if constexpr (!std::is_same<OutT, int>::value) {
            ws = e.w_scale[n];
            if (NB == 2) ws_up = e.w_scale[N + n];
            if (e.flags & EPI_BIAS) b = (float)e.bias[n];
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * WM + i * 16 + row_base + r;
                if (m >= M) continue;
                const size_t at = (size_t)m * N + n;
                if constexpr (std::is_same<OutT, int>::value) {
                    out[at] = acc[0][i][j][r];
                } else {
                    const float xs = e.x_scale[m];
                    float value = ((float)acc[0][i][j][r] * xs) * ws;
                    if (e.flags & EPI_BIAS) value = value + b;
                    if constexpr (NB == 2) {
                        const float up = ((float)acc[1][i][j][r] * xs) * ws_up;
                        value = silu_fast(value) * up;
                    }
                    if (e.flags & EPI_RESIDUAL) value = value + (float)e.residual[at];
                    if (e.flags & EPI_MIX) value = (to_float(from_float<OutT>(value)) * rs) + ((float)e.original[at] * is);
                    out[at] = from_float<OutT>(value);
                }
            }
    }
}

template <int BM, int BN, int NB, typename OutT>
int launch(const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, hipStream_t stream) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((int8_gemm_kernel<BM, BN, NB, OutT>), dim3(tiles), dim3(THREADS), 0, stream, (const int8_t*)x, (const int8_t*)w,
                       (OutT*)out, e, M, N, K);
    return launch_status();
}

// tile 1 is 64 rows, tile 2 is 128; 0 takes the large tile once it fills the chip's 256 CUs twice over.
template <int NB, typename OutT>
int dispatch(const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, int tile, hipStream_t stream) {
    constexpr int BN_LARGE = NB == 2 ? 64 : 128;
    const long large_tiles = (long)((M + 127) / 128) * ((N + BN_LARGE - 1) / BN_LARGE);
    if (tile == 2 || (tile == 0 && large_tiles >= 512)) return launch<128, BN_LARGE, NB, OutT>(x, w, out, e, M, N, K, stream);
    return launch<64, NB == 2 ? 32 : 64, NB, OutT>(x, w, out, e, M, N, K, stream);
}

int check(const void* x, const void* w, void* out, int M, int N, int K, const char* what) {
    if (M < 0 || N <= 0 || K <= 0) return chess_fail(CHESS_INVALID_SHAPE, "%s: M %d, N %d, K %d", what, M, N, K);
    if (K % BK != 0) return chess_fail(CHESS_INVALID_SHAPE, "%s reads the %d inputs %d at a time", what, K, BK);
    if (!x || !w || !out) return chess_fail(CHESS_INVALID_SHAPE, "%s: a required pointer is null", what);
    if (!aligned16(x) || !aligned16(w)) return chess_fail(CHESS_MISALIGNED, "%s's 16-byte loads need aligned x and w", what);
    return CHESS_OK;
}

}  // namespace

extern "C" int chess_int8_linear(const void* x, const void* x_scale, const void* w, const void* w_scale, const void* bias,
                                 const void* residual, const void* original, const void* residual_scale, const void* input_scale,
                                 void* out, int M, int N, int K, int gated, int out_dtype, int tile,
                                 void* stream)
{
    if (int status = check(x, w, out, M, N, K, "int8_linear")) return status;
    if (!x_scale || !w_scale) return chess_fail(CHESS_INVALID_SHAPE, "int8_linear needs both scales");
    if (original && (!residual_scale || !input_scale))
        return chess_fail(CHESS_INVALID_SHAPE, "int8_linear's input mix needs the residual and input scales");
    if (out_dtype != OUT_F16 && out_dtype != OUT_BF16) return chess_fail(CHESS_UNSUPPORTED, "int8_linear writes fp16 or bf16, not %d", out_dtype);
    if (tile < 0 || tile > 2) return chess_fail(CHESS_UNSUPPORTED, "tile %d is none of 0 (by size), 1 (64 rows), 2 (128 rows)", tile);
    if (M == 0) return CHESS_OK;
    Epilogue e{(const float*)x_scale, (const float*)w_scale, (const half_t*)bias, (const half_t*)residual, (const half_t*)original,
               (const half_t*)residual_scale, (const half_t*)input_scale,
               (bias ? EPI_BIAS : 0) | (residual ? EPI_RESIDUAL : 0) | (original ? EPI_MIX : 0)};
    hipStream_t s = (hipStream_t)stream;
    if (gated) {
        return out_dtype == OUT_F16 ? dispatch<2, half_t>(x, w, out, e, M, N, K, tile, s) : dispatch<2, bf16_t>(x, w, out, e, M, N, K, tile, s);
    }
    return out_dtype == OUT_F16 ? dispatch<1, half_t>(x, w, out, e, M, N, K, tile, s) : dispatch<1, bf16_t>(x, w, out, e, M, N, K, tile, s);
}

extern "C" int chess_int8_matmul_i32(const void* x, const void* w, void* out, int M, int N, int K, int tile, void* stream)
{
    if (int status = check(x, w, out, M, N, K, "int8_matmul_i32")) return status;
    if (tile < 0 || tile > 2) return chess_fail(CHESS_UNSUPPORTED, "tile %d is none of 0 (by size), 1 (64 rows), 2 (128 rows)", tile);
    if (M == 0) return CHESS_OK;
    Epilogue e{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0};
    return dispatch<1, int>(x, w, out, e, M, N, K, tile, (hipStream_t)stream);
}
