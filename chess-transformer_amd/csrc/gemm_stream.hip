// The gated int8 GEMM (the MLP's gate_up) as a persistent, software-pipelined kernel, for launches with many times
// more output tiles than CUs:
//   out[M, N] = silu((f32(x @ w_gate^T) * x_scale) * w_scale_gate) * ((f32(x @ w_up^T) * x_scale) * w_scale_up)
// x [M, K] and w [2N, K] int8 (the gate's rows, then up's), exact int32 sums, fp16 out -- gemm.hip's gated epilogue
// op for op (model/int8_blocks.py:66-144 of the reference), so it gives the same bits as every other tile.
//
// One workgroup a CU, four wavefronts, 256 x 64 output tiles (a wavefront 64 rows x 64 outputs from 128 weight rows:
// 2 x 2 gate and 2 x 2 up MFMA fragments of v_mfma_i32_32x32x32_i8). The workgroups walk the tiles in turns, an XCD's
// workgroups taking one row block's column tiles together, so that the row block and the weights stay in its L2.
// What the one-tile-a-workgroup kernel cannot do:
//  - the DMA ring of K stages runs on across tile boundaries, so a tile's first stages land while the previous
//    tile multiplies;
//  - a tile's epilogue (dequantise, SiLU * up, round, store: about 13 VALU instructions an output) is cut into one
//    chunk per K step of the next tile and issued among that step's MFMAs, whose issue leaves the VALU idle. The sums
//    of two tiles are alive at once, in the accumulation registers (AGPRs: this file is built without the VGPR form
//    of the MFMAs).
// Operands and outputs go through buffer resources based at the tile: rows past M read as zero, and the stores of
// rows past M are dropped by the hardware's range check. A wavefront stages its 64 output rows in LDS (no barrier:
// the rows are its own) and stores them as whole 128-byte rows, non-temporally, one 16-byte store a lane a step.
//
// Measured on an MI355X at the batch-1024 gate_up (71,680 x 2,048 from 512) it is correct to the bit but slower
// than the 256 x 64 tile at three workgroups a CU (tile 10), and so not in the tile table: with one wavefront a SIMD
// nothing covers the LDS latency of a step, and a step moves about 84 KB through a CU's LDS (operands, scales,
// staging and the DMA's writes) -- more than its MFMAs take at 128 bytes a clock. It stays selectable as tile 12.
#include "chess_common.h"
#include "lds_dma.h"

namespace {

constexpr int BM = 256, BN = 64, NB = 2, WAVES = 4, WM = BM / WAVES, FM = WM / 32, FN = BN / 32;
constexpr int THREADS = 64 * WAVES;
constexpr int BLOCK = 1024;   // bytes a DMA instruction writes: 16 rows x 64 bytes
constexpr int STAGE_K = 64;   // bytes of K a stage
constexpr int A_BLOCKS = BM / 16, B_BLOCKS = NB * BN / 16, BLOCKS = A_BLOCKS + B_BLOCKS, PER_WAVE = BLOCKS / WAVES;
constexpr int STAGE_BYTES = BLOCKS * BLOCK;
// a tile's f32 weight scales (gate, then up) and row scales, then a spare slot for each thread past the weight scales
constexpr int VECTORS = NB * BN + BM + (THREADS - NB * BN);
constexpr int STAGED_ROW = BN * 2 + 16;   // bytes a staged output row
static_assert(BLOCKS % WAVES == 0 && NB * BN <= THREADS && BM == THREADS, "tile shape");

typedef int v16i __attribute__((ext_vector_type(16)));

template <int STAGES, int STEPS>
__global__ __launch_bounds__(THREADS, 1) void gated_stream_kernel(
    const int8_t* __restrict__ x, const int8_t* __restrict__ w, half_t* __restrict__ out, const float* __restrict__ x_scale,
    const float* __restrict__ w_scale, int M, int N, int tiles_n, int tiles)
{
    static_assert(STEPS % STAGES == 0, "a tile's steps fill whole turns of the ring");
    constexpr int K = STEPS * STAGE_K;
    extern __shared__ __align__(16) int8_t lds[];
    LDS_SPACE int8_t* ring = (LDS_SPACE int8_t*)lds;
    // a tile's vectors by its parity in the run, an array of their own: reads of the ring's object would wait for
    // every DMA load in flight
    __shared__ __align__(16) float vectors[2 * VECTORS];
    // each wavefront's 64 output rows, staged so that they leave as whole rows (a row padded to 144 bytes)
    __shared__ __align__(16) int8_t staging[WAVES * WM * STAGED_ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // The run's tiles: turn i takes tile i G + this workgroup's place, the places of one XCD's workgroups (the
    // hardware deals workgroups to the 8 XCDs in turn) consecutive, so that at any time an XCD's workgroups share a
    // row block of x and the weights in its L2.
    const int G = gridDim.x, place = blockIdx.x % 8 * (G / 8) + blockIdx.x / 8;
    const int count = (tiles - place + G - 1) / G;
    if (count <= 0) return;

    // a lane's DMA sources in each of the wavefront's blocks, from the tile's first x row / first weight column:
    // row lane / 4 of the block, 16-byte chunk (lane % 4) ^ (lane / 16) (the swizzle gemm.hip's stages use)
    uint32_t source[PER_WAVE];
#pragma unroll
    for (int p = 0; p < PER_WAVE; p++) {
        const int block = wave * PER_WAVE + p;
        const int row = (block < A_BLOCKS ? block : block - A_BLOCKS) * 16 + (lane >> 2);
        const int chunk = ((lane & 3) ^ ((lane >> 4) & 3)) * 16;
        source[p] = block < A_BLOCKS ? (uint32_t)(row * K + chunk) : (uint32_t)(((row / BN) * N + row % BN) * K + chunk);
    }
    // the first row and column of the run's tile `local`
    auto coords = [&](int local) { const int t = local * G + place; return int2{t / tiles_n * BM, t % tiles_n * BN}; };
    // the DMA of step ks of the tile at `tile` into ring stage S
    auto issue = [&](int2 tile, int ks, auto stage_index) {
        constexpr int S = decltype(stage_index)::value;
        const BufferResource xr = buffer_resource(x + (size_t)tile.x * K, (uint32_t)(M - tile.x) * (uint32_t)K);
        const BufferResource wr = buffer_resource(w + (size_t)tile.y * K, (uint32_t)(2 * N - tile.y) * (uint32_t)K);
        const uint32_t k0 = (uint32_t)ks * STAGE_K;
#pragma unroll
        for (int p = 0; p < PER_WAVE; p++)
            buffer_dma16(wave * PER_WAVE + p < A_BLOCKS ? xr : wr, (LDS_SPACE void*)(ring + S * STAGE_BYTES + (wave * PER_WAVE + p) * BLOCK),
                         source[p], k0);
    };

    // a lane's operand addresses in stage 0 (fragment and stage offsets are immediates): an operand lane holds row
    // lane % 32 and 16-byte half lane / 32 of each 32-byte sub-step
    const int in_row = lane & 31, half = lane >> 5, r16 = in_row & 15;
    int a_operand[2], b_operand[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
        const int operand = (in_row >> 4) * BLOCK + (r16 * 4 + ((half + 2 * sub) ^ (r16 >> 2))) * 16;
        a_operand[sub] = operand + (wave * WM / 16) * BLOCK;
        b_operand[sub] = operand + A_BLOCKS * BLOCK;
    }

    v16i acc[2][NB][FM][FN];   // two tiles' sums: [tile parity][gate, up][row fragment][column fragment]
    // the odd parity's, which the first tile's (dropped) epilogue reads, start defined
#pragma unroll
    for (int g = 0; g < NB; g++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[1][g][i][j] = v16i{};

    // a step's operands, both 32-byte sub-steps (read at the top of the step: with one wavefront a SIMD, nothing else
    // covers the LDS latency), then its MFMAs into the sums of parity P; the first step's start from zero sums
    struct Operands { v4i a[2][FM], b[2][NB][FN]; };
    auto load_operands = [&](auto stage_index) {
        constexpr int STAGE = decltype(stage_index)::value * STAGE_BYTES;
        Operands o;
#pragma unroll
        for (int sub = 0; sub < 2; sub++) {
#pragma unroll
            for (int i = 0; i < FM; i++) o.a[sub][i] = *(const LDS_SPACE v4i*)(ring + a_operand[sub] + STAGE + (i * 32 / 16) * BLOCK);
#pragma unroll
            for (int g = 0; g < NB; g++)
#pragma unroll
                for (int j = 0; j < FN; j++) o.b[sub][g][j] = *(const LDS_SPACE v4i*)(ring + b_operand[sub] + STAGE + ((g * BN + j * 32) / 16) * BLOCK);
        }
        return o;
    };
    auto multiply = [&](auto parity, const Operands& o, auto first_step) {
        constexpr int P = decltype(parity)::value;
        constexpr bool FIRST = decltype(first_step)::value;
#pragma unroll
        for (int sub = 0; sub < 2; sub++)
#pragma unroll
            for (int g = 0; g < NB; g++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int i = 0; i < FM; i++)
                        acc[P][g][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.b[sub][g][j], o.a[sub][i], FIRST && sub == 0 ? v16i{} : acc[P][g][i][j], 0, 0, 0);
    };

    // chunk C (of STEPS) of the epilogue of the run's tile `local`, whose sums have parity P: 64 outputs a lane,
    // 64 / STEPS a chunk. A lane's sums of fragment (i, j) are row in_row, columns 8 q + 4 half + r in register 4 q + r.
    static_assert(FM * FN * 4 % STEPS == 0, "whole quads a chunk");
    constexpr int QUADS = FM * FN * 4 / STEPS;
    // Run for local = -1 too (before the first tile), unconditionally so that it can be scheduled among the MFMAs:
    // its stores then go through a resource of no bytes, which drops them.
    static_assert(QUADS == 2, "a chunk's two quads share a row fragment");
    constexpr int FRAGMENT_QUADS = 4;
    struct Scales { float xs; v4f ws[QUADS], ws_up[QUADS]; v4u rows; };
    // the chunk's scales, read as one group with its own wait (the compiler would wait for the DMA in flight too);
    // issued at the top of a step, so that the chunk's arithmetic can go among the step's MFMAs
    // the lane's bases: its row's row scale, its quad half's weight scales (the rest are immediate offsets)
    const uint32_t vectors_base = (uint32_t)(uintptr_t)(const LDS_SPACE float*)vectors;
    const uint32_t xs_base = vectors_base + (NB * BN + wave * WM + in_row) * 4, ws_base = vectors_base + 4 * half * 4;
    // and, in the same group, part `part` of the staged rows: 8 rows of 128 bytes, 16 a lane
    const uint32_t staging_base = (uint32_t)(uintptr_t)(const LDS_SPACE int8_t*)staging + wave * WM * STAGED_ROW;
    const uint32_t read_base = staging_base + (lane / 8) * STAGED_ROW + (lane % 8) * 16;
    auto epilogue_scales = [&](auto parity, auto chunk, auto part) {
        constexpr int P = decltype(parity)::value, C = decltype(chunk)::value, I = C * QUADS / (FN * FRAGMENT_QUADS);
        constexpr int PART = decltype(part)::value * 8 * STAGED_ROW;
        constexpr int Q0 = C * QUADS, Q1 = Q0 + 1;   // the chunk's quads (i, j, q), q fastest
        constexpr int XS = (P * VECTORS + I * 32) * 4;
        constexpr int WS0 = (P * VECTORS + Q0 / FRAGMENT_QUADS % FN * 32 + 8 * (Q0 % FRAGMENT_QUADS)) * 4;
        constexpr int WS1 = (P * VECTORS + Q1 / FRAGMENT_QUADS % FN * 32 + 8 * (Q1 % FRAGMENT_QUADS)) * 4;
        Scales scales;
        asm volatile("ds_read_b32 %0, %6 offset:%9\n\tds_read_b128 %1, %7 offset:%10\n\tds_read_b128 %2, %7 offset:%11\n\t"
                     "ds_read_b128 %3, %7 offset:%12\n\tds_read_b128 %4, %7 offset:%13\n\tds_read_b128 %5, %8 offset:%14\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=v"(scales.xs), "=v"(scales.ws[0]), "=v"(scales.ws_up[0]), "=v"(scales.ws[1]), "=v"(scales.ws_up[1]), "=v"(scales.rows)
                     : "v"(xs_base), "v"(ws_base), "v"(read_base), "i"(XS), "i"(WS0), "i"(WS0 + BN * 4), "i"(WS1), "i"(WS1 + BN * 4), "i"(PART)
                     : "memory");
        return scales;
    };
    // a lane's place in the staged rows (its row, its quad half) and in the output (part rows and columns, 16 bytes)
    const uint32_t write_base = staging_base + in_row * STAGED_ROW + half * 8;
    const uint32_t out_base = (uint32_t)(((wave * WM + lane / 8) * N + (lane % 8) * 8) * 2);
    // part `part` (8 rows) of the staged rows of the tile at `tile` to the output, whole rows
    auto store_rows = [&](const v4u& rows, auto part, int2 tile, bool valid) {
        const BufferResource to = buffer_resource(out + (size_t)tile.x * N, valid ? (uint32_t)(M - tile.x) * (uint32_t)N * 2 : 0u);
        buffer_store16_streamed(to, rows, out_base, (uint32_t)(tile.y + decltype(part)::value * 8 * N) * 2);
    };
    auto epilogue = [&](auto parity, auto chunk, const Scales& scales) {
        constexpr int P = decltype(parity)::value, C = decltype(chunk)::value;
        const float xs = scales.xs;
        const uint32_t to = write_base;
#pragma unroll
        for (int u = 0; u < QUADS; u++) {
            const int quad_index = C * QUADS + u;                 // (i, j, q), q fastest
            const int i = quad_index / (FN * FRAGMENT_QUADS), j = quad_index / FRAGMENT_QUADS % FN, q = quad_index % FRAGMENT_QUADS;
            const v4f ws = scales.ws[u], ws_up = scales.ws_up[u];
            const float ws_r[4] = {ws[0], ws[1], ws[2], ws[3]}, ws_up_r[4] = {ws_up[0], ws_up[1], ws_up[2], ws_up[3]};
            half_t value[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float gate = ((float)acc[P][0][i][j][4 * q + r] * xs) * ws_r[r];
                const float up = ((float)acc[P][1][i][j][4 * q + r] * xs) * ws_up_r[r];
                value[r] = (half_t)(silu_fast(gate) * up);
            }
            const v2u packed = __builtin_bit_cast(v2u, v4h{value[0], value[1], value[2], value[3]});
            asm volatile("ds_write_b64 %0, %1 offset:%2" : : "v"(to), "v"(packed), "i"((i * 32) * STAGED_ROW + (j * 32 + 8 * q) * 2) : "memory");
        }
    };

    // a tile's vectors: loaded (raw bits) at its first step, parked in LDS at a later one, read by its epilogue
    // during the next tile, after that tile's barriers
    uint32_t loaded[2];
    auto load_vectors = [&](int2 tile) {
        const int m0 = tile.x, n0 = tile.y;
        // unconditional loads from chosen places (a load under a divergent branch would be waited for early)
        loaded[0] = __float_as_uint(w_scale[tid < NB * BN ? (tid / BN) * N + n0 + tid % BN : 0]);
        loaded[1] = __float_as_uint(x_scale[min(m0 + tid, M - 1)]);
    };
    auto park_vectors = [&](auto parity) {
        constexpr int P = decltype(parity)::value;
        // unconditional (a conditional store would draw the load down to it, and wait for it there)
        LDS_SPACE float* to = (LDS_SPACE float*)vectors + P * VECTORS;
        to[tid < NB * BN ? tid : BM + tid] = __uint_as_float(loaded[0]);
        to[NB * BN + tid] = __uint_as_float(loaded[1]);
    };

    // One tile of the run, parity P: its steps, each (after the barrier that says its stage has landed and the
    // stage it refills is read) issuing the DMA STAGES - 1 steps ahead, its MFMAs, and a chunk of the previous
    // tile's epilogue.
    // Staged rows leave a half tile at a time: rows 0-31 of a wavefront's 64 (chunks 0-3) in steps 4-7, rows 32-63
    // (chunks 4-7) in steps 0-3 of the next tile -- while the other half is being written.
    auto tile_pass = [&](auto parity, int local) {
        constexpr int P = decltype(parity)::value;
        const int2 here = coords(local), prev = coords(max(local - 1, 0)), older = coords(max(local - 2, 0)), next = coords(min(local + 1, count - 1));
        const bool more = local + 1 < count;
        load_vectors(here);
        static_for<0, STEPS>([&](auto step_index) {
            constexpr int KS = decltype(step_index)::value, S = KS % STAGES, TARGET = KS + STAGES - 1;
            // This step's DMA was issued STAGES - 1 steps ago. Issued after it, and left in flight: the DMA of the
            // STAGES - 2 steps between, the row store of each of the STAGES - 1 steps since, and the tile's two
            // vector loads while they are younger (the first STAGES - 1 steps).
            stage_barrier<PER_WAVE * (STAGES - 2) + 1 * (STAGES - 1) + (KS < STAGES - 1 ? 2 : 0)>();
            // the DMA STAGES - 1 steps ahead: this tile's, or the next tile's (past the run's end, this tile's last
            // step again)
            if constexpr (TARGET < STEPS) {
                issue(here, TARGET, std::integral_constant<int, TARGET % STAGES>{});
            } else {
                issue(more ? next : here, more ? TARGET - STEPS : STEPS - 1, std::integral_constant<int, TARGET % STAGES>{});
            }
            const Operands operands = load_operands(std::integral_constant<int, S>{});
            constexpr int PART = KS % 4, ROWS_PART = (KS < 4 ? 4 : 0) + PART;   // rows 32-63 of two tiles back, then 0-31 of the last
            const Scales scales = epilogue_scales(std::integral_constant<int, 1 - P>{}, step_index, std::integral_constant<int, ROWS_PART>{});   // waits for both
            multiply(parity, operands, std::integral_constant<bool, KS == 0>{});
            if constexpr (KS < 4) {
                store_rows(scales.rows, std::integral_constant<int, ROWS_PART>{}, older, local > 1);
            } else {
                store_rows(scales.rows, std::integral_constant<int, ROWS_PART>{}, prev, local > 0);
            }
            epilogue(std::integral_constant<int, 1 - P>{}, step_index, scales);
            if constexpr (KS == 1) park_vectors(parity);
            // an MFMA, then a share of the epilogue's VALU work, while it runs
            static_for<0, 2 * NB * FM * FN>([&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
            });
        });
    };

    // the first tile's first stages, each followed by the stores a step issues (dropped: a resource of no bytes), so
    // that the barriers' counts of the memory operations in flight hold from the first step on
    const BufferResource nowhere = buffer_resource(out, 0u);
    static_for<0, STAGES - 1>([&](auto s) {
        issue(coords(0), min((int)decltype(s)::value, STEPS - 1), s);
        asm volatile("" ::: "memory");   // in this order, as in a step (where the scales' read keeps it)
        buffer_store16_streamed(nowhere, v4u{0, 0, 0, 0}, 0u, 0u);
        asm volatile("" ::: "memory");
    });
    int local = 0;
    for (; local + 1 < count; local += 2) {
        tile_pass(std::integral_constant<int, 0>{}, local);
        tile_pass(std::integral_constant<int, 1>{}, local + 1);
    }
    // After the last tile (`last`, parity P): the rows 32-63 of the tile before it still staged, then the last tile's
    // epilogue alone, its rows leaving after chunks 3 and 7.
    auto read_rows = [&](auto part) {
        v4u rows;
        asm volatile("ds_read_b128 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(rows) : "v"(read_base), "i"(decltype(part)::value * 8 * STAGED_ROW) : "memory");
        return rows;
    };
    auto finish = [&](auto parity, int last) {
        const int2 tile = coords(last), before = coords(max(last - 1, 0));
        __builtin_amdgcn_s_waitcnt(LGKMCNT_ZERO);   // and a barrier: the last tile's parked vectors are visible
        bare_barrier();
        static_for<4, 8>([&](auto part) { store_rows(read_rows(part), part, before, last > 0); });
        static_for<0, STEPS>([&](auto c) {
            epilogue(parity, c, epilogue_scales(parity, c, std::integral_constant<int, 0>{}));
            if constexpr (decltype(c)::value == 3) static_for<0, 4>([&](auto part) { store_rows(read_rows(part), part, tile, true); });
            if constexpr (decltype(c)::value == 7) static_for<4, 8>([&](auto part) { store_rows(read_rows(part), part, tile, true); });
        });
    };
    if (local < count) {
        tile_pass(std::integral_constant<int, 0>{}, local);
        finish(std::integral_constant<int, 0>{}, local);
    } else {
        finish(std::integral_constant<int, 1>{}, local - 1);
    }
    __builtin_amdgcn_s_waitcnt(0);   // the tail's repeated DMA loads land before the workgroup's LDS is released
}

int stream_cus = 0;

}  // namespace

// Launches the persistent gated GEMM; the caller (gemm.hip's chess_int8_linear) has checked the operands.
// K must be 512 and N a multiple of 64.
int launch_gated_stream(const void* x, const void* w, void* out, const float* x_scale, const float* w_scale, int M, int N, int K,
                        hipStream_t stream)
{
    constexpr int STAGES = 4, STEPS = 8;
    if (K != STEPS * STAGE_K || N % BN != 0) return chess_fail(CHESS_UNSUPPORTED, "the streamed gated GEMM takes K = %d and N a multiple of %d, not K = %d, N = %d", STEPS * STAGE_K, BN, K, N);
    if ((uint64_t)M * N * 2 >= (1ull << 32)) return chess_fail(CHESS_UNSUPPORTED, "the streamed gated GEMM addresses its output in 32 bits: %d x %d is too large", M, N);
    if (M == 0) return CHESS_OK;
    if (stream_cus == 0) {
        int device = 0, cus = 0;
        hipError_t error = hipGetDevice(&device);
        if (error == hipSuccess) error = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (error != hipSuccess) return (int)error;
        stream_cus = cus;
    }
    constexpr int BYTES = STAGES * STAGE_BYTES;   // and the vectors' static 3 KB
    auto kernel = gated_stream_kernel<STAGES, STEPS>;
    static const hipError_t allowed = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, BYTES);
    if (allowed != hipSuccess) return (int)allowed;
    const int tiles_n = N / BN, tiles = ((M + BM - 1) / BM) * tiles_n;
    const int blocks = stream_cus / 8 * 8;   // whole XCDs
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(THREADS), BYTES, stream, (const int8_t*)x, (const int8_t*)w, (half_t*)out, x_scale, w_scale, M, N,
                       tiles_n, tiles);
    return launch_status();
}
