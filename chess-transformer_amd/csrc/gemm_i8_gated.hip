// The GEMM's tiles for int8 in, gated (silu(gate) * up), fp16 or bf16 out (gemm_tiles.h), in a translation unit of their own.
#include "gemm_tiles.h"

int gemm::dispatch_i8_gated(int out_dtype, const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, int tile,
                            hipStream_t stream) {
    return out_dtype == OUT_F16 ? dispatch<int8_t, 2, half_t>(x, w, out, e, M, N, K, tile, stream)
                                : dispatch<int8_t, 2, bf16_t>(x, w, out, e, M, N, K, tile, stream);
}
