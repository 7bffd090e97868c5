// Fused template attention over one position's T tokens (64 squares, then T - 64 metadata tokens).
// Computes what model/fused_blocks.py:35-97 (template_bias_kernel + template_attention_kernel) and
// model/attention_cuda.py:97-304 compute, for any head counts and widths:
//   q = f16(RMSNorm_head(q) * q_gain), k = f16(RMSNorm_head(k) * k_gain)    (f32 norms)
//   s[i, j] = (q_i . k_j) * scale + [i, j < 64] f16(sum_t c[b, i, h, t] templates[t, i, j])
//   out_i = sum_j f16(exp(s_ij - max_i)) v_j / sum_j exp(s_ij - max_i)
// projected[B, T, H*dq | KV*dq | KV*dv | H*tc] in, out[B, T, H*dv] (fp16). The templates come key-major,
// keyed[i][j][t] (8 templates a key, zero past templates_count), so that a lane reads its query's
// templates for 4 keys as 4 16-byte loads (the reference pairs its templates likewise,
// model/attention_cuda.py:410-440).
//
// A workgroup takes one position and one or more key/value groups; it has one wavefront per slab of
// 16 queries. For each group the workgroup stages the normalised keys [key][dq] and the values,
// transposed, [d][key] in LDS. A wavefront then runs each head of the group on v_mfma_f32_16x16x32_f16:
// the scores come out transposed, S^T = K Q^T, so a lane holds one query's scores for 4 keys of each
// 16-key tile -- exactly the fragment O^T = V^T P^T needs as its B operand, so the probabilities
// never leave registers. A lane keeps its query's templates for its 16 square keys in registers across
// the heads, as f16 pairs: the bias of a key is 4 v_dot2_f32_f16 of them with the head's coefficients.
#include "chess_common.h"

namespace {

constexpr int MAX_TEMPLATES = 8;
constexpr float LOG2E = 1.44269504f;

typedef __fp16 h2 __attribute__((ext_vector_type(2)));

DEVICE float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
}

// TILES: key tiles of 16 the instantiation holds (T <= 16 TILES)
template <int DQP, int DV, int TILES>
struct Layout {
    static constexpr int STEPS = (TILES + 1) / 2;     // 32-key steps of P V
    static constexpr int KEYS = TILES * 16;           // keys staged
    static constexpr int VKEYS = STEPS * 32;          // value keys staged (zero past T)
    static constexpr int K_ROW = DQP + 8;             // halves a staged key, padded against bank conflicts
    static constexpr int V_ROW = VKEYS + 8;           // halves a staged value column: 8 mod 16, so that the
                                                      // transposing writes of key pairs spread over the banks
};

template <int DQP, int DV, int TILES>
__global__ __launch_bounds__(64 * TILES) void template_attention_kernel(
    const half_t* __restrict__ projected, const half_t* __restrict__ keyed, const half_t* __restrict__ q_gain,
    const half_t* __restrict__ k_gain, half_t* __restrict__ out, int T, int heads, int kv_heads, int dq, int templates_count,
    int groups_per_block, float eps, float scale)
{
    typedef Layout<DQP, DV, TILES> L;
    __shared__ __align__(16) half_t keys[L::KEYS * L::K_ROW];
    __shared__ __align__(16) half_t values[DV * L::V_ROW];

    const int lane = threadIdx.x & 63, slab = threadIdx.x >> 6;
    const int threads = blockDim.x;
    const int b = blockIdx.y;
    const int tiles = (T + 15) / 16;            // key tiles of the scores
    const int width = heads * dq + kv_heads * dq + kv_heads * DV + heads * templates_count;
    const int k_offset = heads * dq, v_offset = k_offset + kv_heads * dq, c_offset = v_offset + kv_heads * DV;
    const int per_kv = heads / kv_heads;
    const half_t* board = projected + (size_t)b * T * width;

    const int col = lane & 15, quad = lane >> 4;
    const int query = slab * 16 + col;
    const bool query_ok = query < T;
    const bool square_query = query < 64;

    // this lane's templates: keyed[query][16 kt + 4 quad + r][0..7], 4 f16 pairs a key
    uint4 pairs[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            pairs[kt][r] = square_query ? *reinterpret_cast<const uint4*>(keyed + ((size_t)query * 64 + kt * 16 + quad * 4 + r) * MAX_TEMPLATES)
                                        : uint4{0, 0, 0, 0};

    half_t q_gains[DQP / 32][8];
#pragma unroll
    for (int ks = 0; ks < DQP / 32; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = ks * 32 + quad * 8 + e;
            q_gains[ks][e] = d < dq ? q_gain[d] : (half_t)0.0f;
        }

    for (int gi = 0; gi < groups_per_block; gi++) {
        const int group = blockIdx.x * groups_per_block + gi;
        if (gi > 0) __syncthreads();   // every wavefront is done with the previous group's keys and values

        // keys: 8-half chunks, CH = DQP / 8 adjacent lanes a key, normalised with the gain
        constexpr int CH = DQP / 8;
        for (int item = threadIdx.x; item < tiles * 16 * CH; item += threads) {
            const int key = item / CH, c = item % CH;
            float v[8];
            if (key < T && c * 8 < dq) {
                const v8h raw = *reinterpret_cast<const v8h*>(board + (size_t)key * width + k_offset + group * dq + c * 8);
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (float)raw[e];
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = 0.0f;
            }
            float squares = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) squares += v[e] * v[e];
#pragma unroll
            for (int offset = 1; offset < CH; offset <<= 1) squares += __shfl_xor(squares, offset, 64);
            const float inverse = 1.0f / __builtin_sqrtf(squares / (float)dq + eps);
            v8h normed;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = c * 8 + e;
                normed[e] = (half_t)(d < dq ? (v[e] * inverse) * (float)k_gain[d] : 0.0f);
            }
            *reinterpret_cast<v8h*>(keys + key * L::K_ROW + c * 8) = normed;
        }
        // values, transposed to [d][key] a key pair at a time (4-byte writes); keys past T are zero
        constexpr int VC = DV / 8, KP = L::VKEYS / 2;
        for (int item = threadIdx.x; item < KP * VC; item += threads) {
            const int kp = item % KP, c = item / KP, key = 2 * kp;
            v8h first = v8h{0, 0, 0, 0, 0, 0, 0, 0}, second = v8h{0, 0, 0, 0, 0, 0, 0, 0};
            if (key < T) first = *reinterpret_cast<const v8h*>(board + (size_t)key * width + v_offset + group * DV + c * 8);
            if (key + 1 < T) second = *reinterpret_cast<const v8h*>(board + (size_t)(key + 1) * width + v_offset + group * DV + c * 8);
            const uint4 lo = __builtin_bit_cast(uint4, first), hi = __builtin_bit_cast(uint4, second);
            const uint32_t lo_words[4] = {lo.x, lo.y, lo.z, lo.w}, hi_words[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                // element e of a row is half e % 2 of its word e / 2
                const uint32_t a = e % 2 ? lo_words[e / 2] >> 16 : lo_words[e / 2] & 0xFFFFu;
                const uint32_t b = e % 2 ? hi_words[e / 2] >> 16 : hi_words[e / 2] & 0xFFFFu;
                *reinterpret_cast<uint32_t*>(values + (c * 8 + e) * L::V_ROW + key) = a | (b << 16);
            }
        }
        __syncthreads();

        for (int hi = 0; hi < per_kv; hi++) {
            const int head = group * per_kv + hi;
            // the query row's fragment of B: lane holds dq columns ks * 32 + 8 quad .. + 8
            float qv[DQP / 32][8];
            float squares = 0.0f;
#pragma unroll
            for (int ks = 0; ks < DQP / 32; ks++) {
                const int d0 = ks * 32 + quad * 8;
                if (query_ok && d0 < dq) {
                    const v8h raw = *reinterpret_cast<const v8h*>(board + (size_t)query * width + head * dq + d0);
#pragma unroll
                    for (int e = 0; e < 8; e++) qv[ks][e] = (float)raw[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) qv[ks][e] = 0.0f;
                }
#pragma unroll
                for (int e = 0; e < 8; e++) squares += qv[ks][e] * qv[ks][e];
            }
            // this query's template coefficients for the head, as f16 pairs (zero past templates_count)
            uint4 coefficients = uint4{0, 0, 0, 0};
            if (square_query) {
                const half_t* from = board + (size_t)query * width + c_offset + head * templates_count;
                if (templates_count == MAX_TEMPLATES) {
                    coefficients = *reinterpret_cast<const uint4*>(from);
                } else {
                    uint16_t c[MAX_TEMPLATES];
#pragma unroll
                    for (int t = 0; t < MAX_TEMPLATES; t++) c[t] = t < templates_count ? __builtin_bit_cast(uint16_t, from[t]) : (uint16_t)0;
                    coefficients = uint4{c[0] | ((uint32_t)c[1] << 16), c[2] | ((uint32_t)c[3] << 16), c[4] | ((uint32_t)c[5] << 16),
                                         c[6] | ((uint32_t)c[7] << 16)};
                }
            }
            squares += __shfl_xor(squares, 16, 64);
            squares += __shfl_xor(squares, 32, 64);
            const float q_inverse = 1.0f / __builtin_sqrtf(squares / (float)dq + eps);
            v8h qf[DQP / 32];
#pragma unroll
            for (int ks = 0; ks < DQP / 32; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) qf[ks][e] = (half_t)((qv[ks][e] * q_inverse) * (float)q_gains[ks][e]);

            // S^T tiles: lane holds s[query][16 kt + 4 quad + r]
            float s[2 * L::STEPS][4];
            float top = -__builtin_inff();
#pragma unroll
            for (int kt = 0; kt < 2 * L::STEPS; kt++) {
                if (kt >= TILES || kt >= tiles) {
#pragma unroll
                    for (int r = 0; r < 4; r++) s[kt][r] = -__builtin_inff();
                    continue;
                }
                v4f acc = v4f{0, 0, 0, 0};
#pragma unroll
                for (int ks = 0; ks < DQP / 32; ks++) {
                    const v8h kf = *reinterpret_cast<const v8h*>(keys + (kt * 16 + col) * L::K_ROW + ks * 32 + quad * 8);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], acc, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = kt * 16 + quad * 4 + r;
                    float value = acc[r] * scale;
                    if (kt < 4 && square_query) {
                        float bias = dot2(coefficients.x, pairs[kt][r].x, 0.0f);
                        bias = dot2(coefficients.y, pairs[kt][r].y, bias);
                        bias = dot2(coefficients.z, pairs[kt][r].z, bias);
                        bias = dot2(coefficients.w, pairs[kt][r].w, bias);
                        value += (float)(half_t)bias;
                    }
                    s[kt][r] = key < T ? value : -__builtin_inff();
                    top = fmaxf(top, s[kt][r]);
                }
            }
            top = fmaxf(top, __shfl_xor(top, 16, 64));
            top = fmaxf(top, __shfl_xor(top, 32, 64));
            float total = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2 * L::STEPS; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = kt < TILES ? __builtin_amdgcn_exp2f((s[kt][r] - top) * LOG2E) : 0.0f;
                    s[kt][r] = p;
                    total += p;
                }
            total += __shfl_xor(total, 16, 64);
            total += __shfl_xor(total, 32, 64);
            const float inverse_total = 1.0f / total;

            // O^T = V^T P^T over 32-key steps: position e of both operands is key 32 st + 16 (e / 4) + 4 quad + e % 4
            v4f o[DV / 16];
#pragma unroll
            for (int dt = 0; dt < DV / 16; dt++) o[dt] = v4f{0, 0, 0, 0};
#pragma unroll
            for (int st = 0; st < L::STEPS; st++) {
                if (2 * st >= tiles) break;
                v8h pf;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    pf[r] = (half_t)s[2 * st][r];
                    pf[4 + r] = (half_t)s[2 * st + 1][r];
                }
#pragma unroll
                for (int dt = 0; dt < DV / 16; dt++) {
                    const half_t* row = values + (dt * 16 + col) * L::V_ROW + st * 32 + quad * 4;
                    const v4h lo = *reinterpret_cast<const v4h*>(row);
                    const v4h hi = *reinterpret_cast<const v4h*>(row + 16);
                    const v8h vf = v8h{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[dt], 0, 0, 0);
                }
            }
            if (query_ok) {
                half_t* to = out + ((size_t)b * T + query) * (heads * DV) + head * DV + quad * 4;
#pragma unroll
                for (int dt = 0; dt < DV / 16; dt++) {
                    const v4h result = v4h{(half_t)(o[dt][0] * inverse_total), (half_t)(o[dt][1] * inverse_total),
                                           (half_t)(o[dt][2] * inverse_total), (half_t)(o[dt][3] * inverse_total)};
                    *reinterpret_cast<v4h*>(to + dt * 16) = result;
                }
            }
        }
    }
}

template <int DQP, int DV, int TILES>
int launch(const void* projected, const void* keyed, const void* q_gain, const void* k_gain, void* out, int B, int T, int heads,
           int kv_heads, int dq, int templates_count, int groups_per_block, float eps, float scale, hipStream_t stream)
{
    const dim3 grid(kv_heads / groups_per_block, B), block(64 * ((T + 15) / 16));
    hipLaunchKernelGGL((template_attention_kernel<DQP, DV, TILES>), grid, block, 0, stream, (const half_t*)projected, (const half_t*)keyed,
                       (const half_t*)q_gain, (const half_t*)k_gain, (half_t*)out, T, heads, kv_heads, dq, templates_count, groups_per_block,
                       eps, scale);
    return launch_status();
}

template <int DQP, int DV>
int by_tokens(const void* projected, const void* keyed, const void* q_gain, const void* k_gain, void* out, int B, int T, int heads,
              int kv_heads, int dq, int templates_count, int groups_per_block, float eps, float scale, hipStream_t stream)
{
    if (T <= 64) return launch<DQP, DV, 4>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
    if (T <= 80) return launch<DQP, DV, 5>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
    return launch<DQP, DV, 8>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
}

template <int DQP>
int by_dv(const void* projected, const void* keyed, const void* q_gain, const void* k_gain, void* out, int B, int T, int heads,
          int kv_heads, int dq, int dv, int templates_count, int groups_per_block, float eps, float scale, hipStream_t stream)
{
    switch (dv) {
        case 16: return by_tokens<DQP, 16>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
        case 32: return by_tokens<DQP, 32>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
        case 64: return by_tokens<DQP, 64>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
        default: return by_tokens<DQP, 128>(projected, keyed, q_gain, k_gain, out, B, T, heads, kv_heads, dq, templates_count, groups_per_block, eps, scale, stream);
    }
}

}  // namespace

extern "C" int chess_template_attention(const void* projected, const void* keyed_templates, const void* q_gain, const void* k_gain, void* out,
                                        int B, int T, int heads, int kv_heads, int dq, int dv, int templates_count, int groups_per_block,
                                        float eps, float scale, void* stream)
{
    if (B < 0 || T < 64 || T > 128)
        return chess_fail(CHESS_UNSUPPORTED, "template_attention takes 64 to 128 tokens a position, not %d", T);
    if (heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0)
        return chess_fail(CHESS_INVALID_SHAPE, "%d heads cannot be split into groups for %d key/value heads", heads, kv_heads);
    if (dq <= 0 || dq > 128 || dq % 8 != 0) return chess_fail(CHESS_UNSUPPORTED, "template_attention takes query widths of 8 to 128 in steps of 8, not %d", dq);
    if (dv != 16 && dv != 32 && dv != 64 && dv != 128) return chess_fail(CHESS_UNSUPPORTED, "template_attention takes value widths 16, 32, 64 or 128, not %d", dv);
    if (templates_count < 0 || templates_count > MAX_TEMPLATES)
        return chess_fail(CHESS_UNSUPPORTED, "template_attention takes at most %d templates, not %d", MAX_TEMPLATES, templates_count);
    if (groups_per_block <= 0 || kv_heads % groups_per_block != 0)
        return chess_fail(CHESS_INVALID_SHAPE, "%d key/value groups a workgroup do not divide %d", groups_per_block, kv_heads);
    if (!projected || !keyed_templates || !q_gain || !k_gain || !out) return chess_fail(CHESS_INVALID_SHAPE, "template_attention: a required pointer is null");
    const int width = heads * dq + kv_heads * dq + kv_heads * dv + heads * templates_count;
    if (!aligned16(projected) || !aligned16(out) || !aligned16(keyed_templates) || width % 8 != 0)
        return chess_fail(CHESS_MISALIGNED, "template_attention's vector loads need 16-byte aligned rows (row width %d halves)", width);
    if (B == 0) return CHESS_OK;
    hipStream_t s = (hipStream_t)stream;
    if (dq <= 32) return by_dv<32>(projected, keyed_templates, q_gain, k_gain, out, B, T, heads, kv_heads, dq, dv, templates_count, groups_per_block, eps, scale, s);
    if (dq <= 64) return by_dv<64>(projected, keyed_templates, q_gain, k_gain, out, B, T, heads, kv_heads, dq, dv, templates_count, groups_per_block, eps, scale, s);
    return by_dv<128>(projected, keyed_templates, q_gain, k_gain, out, B, T, heads, kv_heads, dq, dv, templates_count, groups_per_block, eps, scale, s);
}
