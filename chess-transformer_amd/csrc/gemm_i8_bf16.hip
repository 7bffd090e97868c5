// The GEMM's tiles for int8 in, bf16 out, not gated (gemm_tiles.h), in a translation unit of their own.
#include "gemm_tiles.h"

int gemm::dispatch_i8_bf16(const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, int tile, hipStream_t stream) {
    return dispatch<int8_t, 1, bf16_t>(x, w, out, e, M, N, K, tile, stream);
}
