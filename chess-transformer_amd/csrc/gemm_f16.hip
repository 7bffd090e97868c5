// The GEMM's tiles for fp16 in (f32 sums), fp16 or f32 out, gated or not (gemm_tiles.h), in a translation unit of their own.
#include "gemm_tiles.h"

int gemm::dispatch_f16(int gated, int out_dtype, const void* x, const void* w, void* out, const Epilogue& e, int M, int N, int K, int tile,
                       hipStream_t stream) {
    if (gated) {
        return out_dtype == OUT_F16 ? dispatch<half_t, 2, half_t>(x, w, out, e, M, N, K, tile, stream)
                                    : dispatch<half_t, 2, float>(x, w, out, e, M, N, K, tile, stream);
    }
    return out_dtype == OUT_F16 ? dispatch<half_t, 1, half_t>(x, w, out, e, M, N, K, tile, stream)
                                : dispatch<half_t, 1, float>(x, w, out, e, M, N, K, tile, stream);
}
