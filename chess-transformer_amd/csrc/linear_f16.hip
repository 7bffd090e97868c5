// fp16 GEMM with linear_epilogue: the combine_heads projection of every block, and all matmuls
// of the blocks kept in fp16 and of the heads.
// Computes what model/fused_blocks.py:229-318 (linear_kernel) computes: out[M, N] = epilogue(x[M, K] @ w[K, N]),
// x fp16 row-major, w fp16 "in_features x out_features" row-major (gated: the gate's N columns,
// then up's). The reference accumulates fp16 products in fp16 (or fp32 with accumulate_fp32);
// MFMA accumulates in f32 always, the closer answer. Epilogue, in f32:
//   [+ bias[n]]  [gated: silu(out) * up]  [+ residual]  [mix: (f32(round(out)) * rs) + (original * is)]
// then fp16 out, or f32 for accumulate_fp32.
//
// A workgroup of 4 wavefronts takes a BM x BN tile; wavefronts take 16x16 fragments of
// v_mfma_f32_16x16x32_f16. K advances 32 at a time through double-buffered LDS. w's tile is stored
// transposed ([n][k]) as it is staged, so that both operands are read from LDS as 16-byte rows.
#include "chess_common.h"

#include <type_traits>

namespace {

constexpr int BK = 32;
constexpr int ROW = BK + 8;        // halves per staged row, padded against bank conflicts
constexpr int THREADS = 256;

enum { EPI_BIAS = 1, EPI_RESIDUAL = 2, EPI_MIX = 4 };

struct Epilogue {
    const half_t* bias;
    const half_t* residual;
    const half_t* original;
    const half_t* residual_scale;
    const half_t* input_scale;
    int flags;
};

template <int BM, int BN, int NB, typename OutT>
__global__ __launch_bounds__(THREADS) void linear_kernel(
    const half_t* __restrict__ x, const half_t* __restrict__ w, OutT* __restrict__ out, Epilogue e, int M, int N, int K)
{
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int A_CHUNKS = BM * BK / 8 / THREADS;
    constexpr int B_CHUNKS = NB * BN * BK / 8 / THREADS;
    constexpr int B_ROW_CHUNKS = NB * BN / 8;   // 8-column chunks along a row of w's tile
    static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for the loaders");
    __shared__ __align__(16) half_t lds_a[2][BM * ROW];
    __shared__ __align__(16) half_t lds_b[2][NB * BN * ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int width = NB * N;

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const int tile = xcd_local_tile(blockIdx.x, tiles_m * tiles_n);
    constexpr int GROUP_M = 8;
    const int in_group = GROUP_M * tiles_n;
    const int first_m = tile / in_group * GROUP_M;
    const int group_rows = min(tiles_m - first_m, GROUP_M);
    const int m0 = (first_m + tile % in_group % group_rows) * BM;
    const int n0 = (tile % in_group / group_rows) * BN;

    const half_t* a_src[A_CHUNKS];
    int a_dst[A_CHUNKS];
#pragma unroll
    for (int c = 0; c < A_CHUNKS; c++) {
        const int idx = tid + c * THREADS, r = idx / (BK / 8), part = idx % (BK / 8);
        a_src[c] = x + (size_t)min(m0 + r, M - 1) * K + part * 8;
        a_dst[c] = r * ROW + part * 8;
    }
    const half_t* b_src[B_CHUNKS];
    int b_row[B_CHUNKS], b_k[B_CHUNKS];
    bool b_ok[B_CHUNKS];
#pragma unroll
    for (int c = 0; c < B_CHUNKS; c++) {
        const int idx = tid + c * THREADS, k = idx / B_ROW_CHUNKS, chunk = idx % B_ROW_CHUNKS;
        const int group = chunk * 8 / BN, n = n0 + chunk * 8 % BN;
        b_ok[c] = n < N;
        b_src[c] = w + (size_t)k * width + group * N + (b_ok[c] ? n : 0);
        b_row[c] = group * BN + chunk * 8 % BN;
        b_k[c] = k;
    }

    uint4 a_reg[A_CHUNKS];
    v8h b_reg[B_CHUNKS];

    v4f acc[NB][FM][FN];
#pragma unroll
    for (int g = 0; g < NB; g++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[g][i][j] = v4f{0, 0, 0, 0};

    const int steps = K / BK;
    const int row_in = lane & 15, part_in = (lane >> 4) * 8;
    {
        const int k0 = 0;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) a_reg[c] = *reinterpret_cast<const uint4*>(a_src[c] + k0);
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++)
            b_reg[c] = b_ok[c] ? *reinterpret_cast<const v8h*>(b_src[c] + (size_t)k0 * width) : v8h{0, 0, 0, 0, 0, 0, 0, 0};
    }
    {
        const int buffer = 0;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_a[buffer][a_dst[c]]) = a_reg[c];
#pragma unroll
        for (int c = 0; c < B_CHUNKS; c++)
#pragma unroll
            for (int i = 0; i < 8; i++) lds_b[buffer][(b_row[c] + i) * ROW + b_k[c]] = b_reg[c][i];
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
            for (int c = 0; c < B_CHUNKS; c++)
                b_reg[c] = b_ok[c] ? *reinterpret_cast<const v8h*>(b_src[c] + (size_t)k0 * width) : v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }
        v8h af[FM];
#pragma unroll
        for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v8h*>(&lds_a[buffer][(wm * WM + i * 16 + row_in) * ROW + part_in]);
#pragma unroll
        for (int g = 0; g < NB; g++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const v8h bf = *reinterpret_cast<const v8h*>(&lds_b[buffer][(g * BN + wn * WN + j * 16 + row_in) * ROW + part_in]);
#pragma unroll
                for (int i = 0; i < FM; i++) acc[g][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf, acc[g][i][j], 0, 0, 0);
            }
        {
            const int next = buffer ^ 1;
#pragma unroll
            for (int c = 0; c < A_CHUNKS; c++) *reinterpret_cast<uint4*>(&lds_a[next][a_dst[c]]) = a_reg[c];
#pragma unroll
            for (int c = 0; c < B_CHUNKS; c++)
#pragma unroll
                for (int i = 0; i < 8; i++) lds_b[next][(b_row[c] + i) * ROW + b_k[c]] = b_reg[c][i];
        }
        __syncthreads();
    }

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
        const float b = (e.flags & EPI_BIAS) ? (float)e.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * WM + i * 16 + row_base + r;
                if (m >= M) continue;
                const size_t at = (size_t)m * N + n;
                float value = acc[0][i][j][r];
                if (e.flags & EPI_BIAS) value = value + b;
                if constexpr (NB == 2) value = silu_fast(value) * acc[1][i][j][r];
                if (e.flags & EPI_RESIDUAL) value = value + (float)e.residual[at];
                if (e.flags & EPI_MIX) value = (to_float(from_float<OutT>(value)) * rs) + ((float)e.original[at] * is);
                out[at] = from_float<OutT>(value);
            }
    }
}

template <int BM, int BN, int NB, typename OutT>
int launch(const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, hipStream_t stream) {
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((linear_kernel<BM, BN, NB, OutT>), dim3(tiles), dim3(THREADS), 0, stream, (const half_t*)x, (const half_t*)w,
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

}  // namespace

extern "C" int chess_linear(const void* x, const void* w, const void* bias, const void* residual, const void* original,
                            const void* residual_scale, const void* input_scale, void* out, int M, int N, int K, int gated, int out_dtype, int tile,
                            void* stream)
{
    if (M < 0 || N <= 0 || K <= 0) return chess_fail(CHESS_INVALID_SHAPE, "linear: M %d, N %d, K %d", M, N, K);
    if (K % BK != 0) return chess_fail(CHESS_INVALID_SHAPE, "linear reads the %d inputs %d at a time", K, BK);
    if (N % 8 != 0) return chess_fail(CHESS_UNSUPPORTED, "linear's 16-byte weight loads need outputs in multiples of 8, not %d", N);
    if (!x || !w || !out) return chess_fail(CHESS_INVALID_SHAPE, "linear: a required pointer is null");
    if (original && (!residual_scale || !input_scale)) return chess_fail(CHESS_INVALID_SHAPE, "linear's input mix needs both scales");
    if (!aligned16(x) || !aligned16(w)) return chess_fail(CHESS_MISALIGNED, "linear's 16-byte loads need aligned x and w");
    if (out_dtype != OUT_F16 && out_dtype != OUT_F32) return chess_fail(CHESS_UNSUPPORTED, "linear writes fp16 or f32, not %d", out_dtype);
    if (tile < 0 || tile > 2) return chess_fail(CHESS_UNSUPPORTED, "tile %d is none of 0 (by size), 1 (64 rows), 2 (128 rows)", tile);
    if (M == 0) return CHESS_OK;
    Epilogue e{(const half_t*)bias, (const half_t*)residual, (const half_t*)original, (const half_t*)residual_scale, (const half_t*)input_scale,
               (bias ? EPI_BIAS : 0) | (residual ? EPI_RESIDUAL : 0) | (original ? EPI_MIX : 0)};
    hipStream_t s = (hipStream_t)stream;
    if (gated) return out_dtype == OUT_F16 ? dispatch<2, half_t>(x, w, out, e, M, N, K, tile, s) : dispatch<2, float>(x, w, out, e, M, N, K, tile, s);
    return out_dtype == OUT_F16 ? dispatch<1, half_t>(x, w, out, e, M, N, K, tile, s) : dispatch<1, float>(x, w, out, e, M, N, K, tile, s);
}
