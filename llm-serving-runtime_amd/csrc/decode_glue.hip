// Decode-step glue on gfx950: KV append into the block pool, rotary embedding fused with the
// append, residual add fused with RMSNorm, and SwiGLU's SiLU * up.
//
// These replace the per-layer torch ops around the int8 linears and the paged-attention
// kernel (the reference runs them as separate HF / torch ops inside every decoder layer,
// and its KV write is a per-token Python loop, runtime/phase2/paged_kv_kernel.py:176-227).
// Every kernel is HBM/latency bound element-wise work: one thread per 16-byte chunk,
// 128-bit loads and stores, no LDS except the RMSNorm row reduction.
#include "common.h"
#include "glue_common.h"

#include <type_traits>

namespace mx {
namespace glue {

constexpr int kThreads = 256;

// Linear output element(s) from split-K partials: fp16(bias[col] + sum_s part[s*split_stride + off]),
// the value mx_w8a16_linear would have written (its reduce adds the bias, then the splits in order).
// KS > 0 is the split count known at compile time: every load is issued before the first add, so
// the partials cost one memory round trip; KS == 0 reads `splits` in a loop.
// The bias is read as one E * 2-byte vector load that is issued whether or not there is a
// bias (from the partials' own first bytes when there is none, then discarded), so no branch
// or wait separates it from the partial loads. Callers keep bias + col aligned to E * 2 bytes.
template <int KS, int E>
__device__ __forceinline__ void sum_splits(const float* part, int splits, int64_t split_stride, int64_t off,
                                           const uint16_t* bias, int col, _Float16 (&out)[E]) {
    using BiasVec = typename std::conditional<E == 8, uint4, uint2>::type;
    static_assert(E == 4 || E == 8, "sum_splits: E is 4 or 8");
    const BiasVec braw = *reinterpret_cast<const BiasVec*>(bias ? bias + col : reinterpret_cast<const uint16_t*>(part));
    _Float16 bv[E];
    __builtin_memcpy(bv, &braw, sizeof(bv));
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = bias ? (float)bv[e] : 0.0f;
    if (KS > 0) {
        float4v v[KS > 0 ? KS : 1][E / 4];
#pragma unroll
        for (int sp = 0; sp < KS; ++sp)
#pragma unroll
            for (int e = 0; e < E; e += 4) v[sp][e / 4] = *reinterpret_cast<const float4v*>(part + sp * split_stride + off + e);
#pragma unroll
        for (int sp = 0; sp < KS; ++sp)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] += v[sp][e / 4][e % 4];
    } else {
        for (int sp = 0; sp < splits; ++sp) {
            const float* q = part + sp * split_stride + off;
#pragma unroll
            for (int e = 0; e < E; e += 4) {
                const float4v v = *reinterpret_cast<const float4v*>(q + e);
                acc[e] += v[0];
                acc[e + 1] += v[1];
                acc[e + 2] += v[2];
                acc[e + 3] += v[3];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) out[e] = (_Float16)pin_f32(acc[e]);
}

struct AppendParams {
    const uint16_t* k_new;
    const uint16_t* v_new;
    int64_t sb, sh, st;  // element strides of the new states [B, Hkv, T, D]
    int T, Hkv, D;
    const int32_t* bt;
    int64_t bt_sb;
    int max_blocks;
    const int32_t* start;
    uint16_t* k_pool;
    uint16_t* v_pool;
    int64_t sblk, shead;
    int bs, num_pool_blocks;
    int32_t* err;
    uint8_t* used;  // optional [num_pool_blocks] map: 1 where a token was written
};

// One thread per 8-element chunk of one (row, token, kv-head); K and V share the slot.
__global__ __launch_bounds__(kThreads) void kv_append_kernel(AppendParams p, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= total) return;
    const int chunks = p.D >> 3;
    const int c = (int)(i % chunks);
    int64_t r = i / chunks;
    const int h = (int)(r % p.Hkv);
    r /= p.Hkv;
    const int t = (int)(r % p.T);
    const int b = (int)(r / p.T);
    const int64_t dst = slot_offset(p.bt, p.bt_sb, p.max_blocks, b, p.start[b] + t, p.bs, p.num_pool_blocks, p.sblk,
                                    p.shead, h, p.D);
    if (dst < 0) {
        if (p.err && c == 0) atomicOr(p.err, 1);
        return;
    }
    const int64_t src = (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)t * p.st + c * 8;
    st16(p.k_pool + dst + c * 8, ld16(p.k_new + src));
    st16(p.v_pool + dst + c * 8, ld16(p.v_new + src));
    // Block-usage accounting (GpuKVBlockPool.allocated_block_count) without a host sync.
    if (p.used && c == 0 && h == 0) p.used[p.bt[(int64_t)b * p.bt_sb + (p.start[b] + t) / p.bs]] = 1;
}

struct RopeAppendParams {
    const uint16_t* qkv;      // fp16 rows, or NULL with part != NULL
    int64_t qkv_stride;
    const float* part;        // split-K partials [splits][B][(Hq + 2 Hkv) * D]
    int splits;
    int64_t split_stride;
    const uint16_t* bias;     // added to the partial sums (NULL: none)
    int Hq, Hkv, D;
    const float2* rope;  // [max_pos][D/2] (cos, sin)
    int max_pos;
    const int32_t* positions;
    uint16_t* q_out;
    int64_t q_stride;
    uint16_t* k_pool;
    uint16_t* v_pool;
    int64_t sblk, shead;
    const int32_t* bt;
    int64_t bt_sb;
    int max_blocks, bs, num_pool_blocks;
    int32_t* err;
    int32_t* lens_out;  // optional: lens_out[b] = positions[b] + 1 (the attention length)
    uint8_t* used;      // optional [num_pool_blocks] map: 1 where a token was written
};

// Rotate-half RoPE (pairs i and i + D/2 share frequency i) on the q and k heads of one
// fused-QKV output row, then q -> q_out and k, v -> the pool slot of position `pos`.
// One thread per 4 pairs of a q/k head (two 8-byte loads) or per 8 elements of a v head.
// KS < 0: fp16 QKV rows; KS >= 0: split partials (see sum_splits).
template <int KS>
__global__ __launch_bounds__(kThreads) void qkv_rope_append_kernel(RopeAppendParams p, int64_t total) {
    constexpr bool SPLIT = KS >= 0;
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= total) return;
    const int per_head = p.D >> 3;
    const int heads = p.Hq + 2 * p.Hkv;
    const int c = (int)(i % per_head);
    const int hs = (int)((i / per_head) % heads);
    const int b = (int)(i / ((int64_t)per_head * heads));
    const uint16_t* row = SPLIT ? nullptr : p.qkv + (int64_t)b * p.qkv_stride + (int64_t)hs * p.D;
    const int64_t poff = SPLIT ? ((int64_t)b * (p.Hq + 2 * p.Hkv) + hs) * p.D : 0;  // element offset in a split
    const int pos = p.positions[b];
    if (p.lens_out && hs == 0 && c == 0) p.lens_out[b] = pos + 1;
    if (hs < p.Hq + p.Hkv) {
        const int half = p.D >> 1;
        const int j = c * 4;
        const bool pos_ok = pos >= 0 && pos < p.max_pos;
        half4v o1 = {0, 0, 0, 0}, o2 = {0, 0, 0, 0};
        if (pos_ok) {
            half4v x1, x2;
            if (SPLIT) {
                _Float16 v1[4], v2[4];
                sum_splits<(KS > 0 ? KS : 0), 4>(p.part, p.splits, p.split_stride, poff + j, p.bias, hs * p.D + j, v1);
                sum_splits<(KS > 0 ? KS : 0), 4>(p.part, p.splits, p.split_stride, poff + half + j, p.bias,
                                                 hs * p.D + half + j, v2);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x1[e] = v1[e];
                    x2[e] = v2[e];
                }
            } else {
                x1 = __builtin_bit_cast(half4v, *reinterpret_cast<const uint2*>(row + j));
                x2 = __builtin_bit_cast(half4v, *reinterpret_cast<const uint2*>(row + half + j));
            }
            const float2* cs = p.rope + (int64_t)pos * half + j;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const half2v o = rope_rotate(x1[e], x2[e], cs[e]);
                o1[e] = o[0];
                o2[e] = o[1];
            }
        } else if (p.err && c == 0) {
            atomicOr(p.err, 2);
        }
        if (hs < p.Hq) {
            uint16_t* q = p.q_out + (int64_t)b * p.q_stride + (int64_t)hs * p.D;
            *reinterpret_cast<uint2*>(q + j) = __builtin_bit_cast(uint2, o1);
            *reinterpret_cast<uint2*>(q + half + j) = __builtin_bit_cast(uint2, o2);
            return;
        }
        if (!pos_ok) return;
        const int64_t dst = slot_offset(p.bt, p.bt_sb, p.max_blocks, b, pos, p.bs, p.num_pool_blocks, p.sblk,
                                        p.shead, hs - p.Hq, p.D);
        if (dst < 0) {
            if (p.err && c == 0) atomicOr(p.err, 1);
            return;
        }
        *reinterpret_cast<uint2*>(p.k_pool + dst + j) = __builtin_bit_cast(uint2, o1);
        *reinterpret_cast<uint2*>(p.k_pool + dst + half + j) = __builtin_bit_cast(uint2, o2);
        if (p.used && c == 0 && hs == p.Hq) p.used[p.bt[(int64_t)b * p.bt_sb + pos / p.bs]] = 1;
        return;
    }
    if (pos >= p.max_pos) return;  // flagged by the q/k threads of the row
    const int64_t dst = slot_offset(p.bt, p.bt_sb, p.max_blocks, b, pos, p.bs, p.num_pool_blocks, p.sblk, p.shead,
                                    hs - p.Hq - p.Hkv, p.D);
    if (dst < 0) return;  // flagged by the k thread of the same chunk
    if (SPLIT) {
        _Float16 v[8];
        sum_splits<(KS > 0 ? KS : 0), 8>(p.part, p.splits, p.split_stride, poff + c * 8, p.bias, hs * p.D + c * 8, v);
        half8v o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[e];
        st16(p.v_pool + dst + c * 8, as_u4(o));
    } else {
        st16(p.v_pool + dst + c * 8, ld16(row + c * 8));
    }
}

// One workgroup per row. 512 threads keep one 8-column chunk per thread at H = 4096, so
// all of a row's split partials (8 x 16 KB at the bench shape) are in flight at once.
constexpr int kNormThreads = 512;
constexpr int kNormMaxChunks = 4;  // H <= kNormThreads * 8 * kNormMaxChunks = 16384

template <int T>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) s += red[w];
    return s;
}

struct NormParams {
    const uint16_t* x;     // fp16 rows, or NULL with part != NULL
    int64_t xs;
    const int64_t* rows;   // optional gather: row m of x is x + rows[m] * xs (an embedding lookup)
    int64_t xcount;        // rows of x a gather may read; an index outside [0, xcount) reads a zero row
    const float* part;     // split-K partials [splits][M][H] of the producing linear
    int splits;
    int64_t split_stride;
    const uint16_t* bias;  // added to the partial sums (NULL: none)
    const uint16_t* res;
    int64_t rs;
    const uint16_t* w;
    int H;
    float eps;
    uint16_t* out;
    int64_t os;
    uint16_t* res_out;
    int64_t ros;
};

// h = x (+ residual, rounded to fp16); residual_out = h; out = fp16(fp16(h * rsqrt(mean(h^2) + eps)) * w).
// The two roundings of the output follow HF's RMSNorm (normalise in fp32, cast, scale in fp16).
// With SPLIT, x is first formed from the producing linear's split partials and rounded to fp16,
// as that linear's own output would have been. out may alias x and residual_out may alias
// residual (each thread reads its chunks before it writes them); out must not alias residual_out.
// KS < 0: fp16 x rows; KS >= 0: split partials (see sum_splits).
template <int KS>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(NormParams p) {
    constexpr bool SPLIT = KS >= 0;
    __shared__ float red[kNormThreads / 64];
    const int m = blockIdx.x;
    const int chunks = p.H >> 3;
    const int64_t xr = SPLIT ? 0 : (p.rows ? p.rows[m] : m);
    const bool x_in = (uint64_t)xr < (uint64_t)p.xcount;
    half8v h[kNormMaxChunks], wv[kNormMaxChunks];
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kNormMaxChunks; ++u) {
        const int c = threadIdx.x + u * kNormThreads;
        if (c < chunks) {
            // Norm weight, residual and x (or its partials) all go out before the first wait;
            // without a residual the residual load re-reads the weights and is discarded.
            wv[u] = as_h8(ld16(p.w + c * 8));
            const half8v r = as_h8(ld16(p.res ? p.res + (int64_t)m * p.rs + c * 8 : p.w + c * 8));
            half8v v;
            if (SPLIT) {
                _Float16 t[8];
                sum_splits<(KS > 0 ? KS : 0), 8>(p.part, p.splits, p.split_stride, (int64_t)m * p.H + c * 8, p.bias,
                                                 c * 8, t);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = t[e];
            } else {
                v = as_h8(ld16(p.x + (x_in ? xr : 0) * p.xs + c * 8));
                if (!x_in) v = half8v{};
            }
            // Without a residual the addend is -0.0, the exact identity of IEEE addition (it
            // keeps -0 as -0), so the load's use, and with it the load, stays unconditional.
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (p.res ? (float)r[e] : -0.0f));
            if (p.res_out) st16(p.res_out + (int64_t)m * p.ros + c * 8, as_u4(v));
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
            h[u] = v;
        }
    }
    const float scale = rsqrtf(block_sum<kNormThreads>(ss, red) / (float)p.H + p.eps);
#pragma unroll
    for (int u = 0; u < kNormMaxChunks; ++u) {
        const int c = threadIdx.x + u * kNormThreads;
        if (c < chunks) {
            const half8v g = wv[u];
            half8v o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 n = (_Float16)((float)h[u][e] * scale);
                o[e] = (_Float16)((float)n * (float)g[e]);
            }
            st16(p.out + (int64_t)m * p.os + c * 8, as_u4(o));
        }
    }
}

// out[m, i] = fp16(fp16(silu(gate[m, i])) * up[m, i]) with gate = gu[m, :I], up = gu[m, I:2I].
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* gu, int64_t gs, int I, uint16_t* out,
                                                            int64_t os, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= total) return;
    const int chunks = I >> 3;
    const int c = (int)(i % chunks);
    const int64_t m = i / chunks;
    const half8v g = as_h8(ld16(gu + m * gs + c * 8));
    const half8v u = as_h8(ld16(gu + m * gs + I + c * 8));
    half8v o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 s = (_Float16)silu_f32((float)g[e]);
        o[e] = (_Float16)((float)s * (float)u[e]);
    }
    st16(out + m * os + c * 8, as_u4(o));
}

// SwiGLU of the interleaved gate||up projection (rows 16t + [0, 8) are gate channels
// 8t + [0, 8), rows 16t + [8, 16) the matching up channels): out[m, 8t + e] =
// fp16(fp16(silu(g)) * u) with g, u rounded to fp16 as the projection's own output is.
// KS < 0: g, u from its fp16 output rows; KS >= 0: from its split-K partials [splits][M][2I]
// plus bias, summed bias-first in split order (bit-identical to mx_w8a16_linear's reduce).
// One thread per (row, group of 8 channels).
template <int KS>
__global__ __launch_bounds__(kThreads) void swiglu_interleaved_kernel(const uint16_t* gu, int64_t gs, const float* part,
                                                                      int splits, const uint16_t* bias, int I,
                                                                      uint16_t* out, int64_t os, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= total) return;
    const int groups = I >> 3;
    const int t = (int)(i % groups);
    const int64_t m = i / groups;
    _Float16 g[8], u[8];
    if (KS < 0) {
        const half8v gv = as_h8(ld16(gu + m * gs + 16 * t));
        const half8v uv = as_h8(ld16(gu + m * gs + 16 * t + 8));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            g[e] = gv[e];
            u[e] = uv[e];
        }
    } else {
        const int64_t n2 = 2 * (int64_t)I, stride = (total / groups) * n2;  // M * 2I per split
        sum_splits<(KS > 0 ? KS : 0), 8>(part, splits, stride, m * n2 + 16 * t, bias, 16 * t, g);
        sum_splits<(KS > 0 ? KS : 0), 8>(part, splits, stride, m * n2 + 16 * t + 8, bias, 16 * t + 8, u);
    }
    half8v o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 sg = (_Float16)silu_f32((float)g[e]);
        o[e] = (_Float16)((float)sg * (float)u[e]);
    }
    st16(out + m * os + 8 * t, as_u4(o));
}

// Chunked greedy argmax (mx_argmax_rows_split): workgroup (c, m) reduces logits
// [c * kArgChunk, (c + 1) * kArgChunk) of row m to one 64-bit key, and one wave per row takes
// the largest key. A key orders (value, index) the way torch.argmax does: the value as an
// order-preserving 17-bit code of the fp16 bits (-0 coded as +0, so they tie; NaN above +inf)
// in the high word, and 0xffffffff - index in the low word, so the larger key of two equal
// values is the earlier index. A row is thus read once, by many CUs: one workgroup per row
// (argmax_kernel below) is bounded by what one CU streams (~50 GB/s), 18.6 us for 16 rows of
// 151936 logits on MI355X.
constexpr int kArgChunk = 4096;
constexpr int kArgChunkThreads = 256;  // 16 logits per thread

__device__ __forceinline__ uint64_t argmax_key(uint32_t bits, uint32_t idx) {
    bits &= 0xffffu;
    const uint32_t mag = bits & 0x7fffu;
    uint32_t ord = (bits & 0x8000u) ? 0x7fffu - mag : 0x8000u + mag;  // -x below +y, larger |x| lower
    ord = mag == 0 ? 0x8000u : ord;                                   // -0 == +0
    ord = mag > 0x7c00u ? 0x10000u : ord;                             // NaN above every number
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)v, o), hi = __shfl_xor((uint32_t)(v >> 32), o);
        v = max_u64(v, ((uint64_t)hi << 32) | lo);
    }
    return v;
}

__global__ __launch_bounds__(kArgChunkThreads) void argmax_chunk_kernel(const uint16_t* __restrict__ logits,
                                                                         int64_t ls, int N, uint64_t* __restrict__ keys,
                                                                         int nchunks) {
    constexpr int kIters = kArgChunk / (8 * kArgChunkThreads);
    const int chunk = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const uint16_t* row = logits + (int64_t)m * ls;
    const int base = chunk * kArgChunk;
    uint4 v[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {  // both loads in flight before the first compare
        const int n0 = base + (it * kArgChunkThreads + tid) * 8;
        v[it] = n0 + 8 <= N ? *reinterpret_cast<const uint4*>(row + n0) : uint4{0, 0, 0, 0};
    }
    uint64_t best = 0;  // below every key: the lowest number (-inf) has code 0x3ff
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int n0 = base + (it * kArgChunkThreads + tid) * 8;
        if (n0 + 8 <= N) {
            const uint32_t w[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                best = max_u64(best, argmax_key(w[j], (uint32_t)(n0 + 2 * j)));
                best = max_u64(best, argmax_key(w[j] >> 16, (uint32_t)(n0 + 2 * j + 1)));
            }
        } else {
            for (int e = 0; e < 8 && n0 + e < N; ++e) best = max_u64(best, argmax_key(row[n0 + e], (uint32_t)(n0 + e)));
        }
    }
    best = wave_max_u64(best);
    __shared__ uint64_t s_best[kArgChunkThreads / 64];
    if ((tid & 63) == 0) s_best[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 1; w < kArgChunkThreads / 64; ++w) best = max_u64(best, s_best[w]);
        keys[(int64_t)m * nchunks + chunk] = best;
    }
}

__global__ __launch_bounds__(64) void argmax_keys_kernel(const uint64_t* __restrict__ keys, int nchunks,
                                                         int64_t* __restrict__ out, int32_t* seq_lens) {
    const int m = blockIdx.x, lane = threadIdx.x;
    uint64_t best = 0;
    for (int c = lane; c < nchunks; c += 64) best = max_u64(best, keys[(int64_t)m * nchunks + c]);
    best = wave_max_u64(best);
    if (lane == 0) {
        out[m] = (int64_t)(0xffffffffu - (uint32_t)best);
        if (seq_lens) seq_lens[m] += 1;
    }
}

// Greedy token of each row: index of the largest logit, the first one on ties; NaN counts as
// larger than any number (torch.argmax's convention). One workgroup of 1024 threads per row.
constexpr int kArgThreads = 1024;
constexpr int kArgU = 16;

// Greedy argmax of one fp16 row in two passes over the row (torch's convention: the
// first index on ties, any NaN counts above every number and the first NaN wins):
//   1. the row maximum with packed fp16 max (v_pk_max_f16, NaNs ignored) and a NaN
//      flag from the bits ((x & 0x7fff) + 0x3ff overflows into bit 15 exactly for NaN);
//   2. the first index whose value equals the maximum (fp16 compare, so -0 == +0), or
//      the first NaN if the row has one.
// About two VALU operations per element per pass; a per-element branchy comparison
// ran at ~20 and made the kernel VALU-bound (22 us for 32 x 128256 on MI355X).
// kArgU chunks of 8 per thread are loaded per memory round trip (indices clamped).
__device__ __forceinline__ uint32_t nan_bits(uint32_t w) { return ((w & 0x7fff7fffu) + 0x03ff03ffu) & 0x80008000u; }

template <typename F>
__device__ __forceinline__ void for_row_chunks(const _Float16* row, int chunks, int tid, F&& f) {
    for (int c0 = tid; c0 < chunks; c0 += kArgU * kArgThreads) {
        uint4 v[kArgU];
#pragma unroll
        for (int u = 0; u < kArgU; ++u) {
            const int c = c0 + u * kArgThreads;
            v[u] = *reinterpret_cast<const uint4*>(row + (c < chunks ? c : chunks - 1) * 8);
        }
#pragma unroll
        for (int u = 0; u < kArgU; ++u) f(c0 + u * kArgThreads, v[u]);
    }
}

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const uint16_t* __restrict__ logits, int64_t ls, int N,
                                                             int64_t* __restrict__ out, int32_t* seq_lens) {
    constexpr int kW = kArgThreads / 64;
    __shared__ float s_max[kW];
    __shared__ int s_nan[kW], s_idx[kW];
    const int m = blockIdx.x, tid = threadIdx.x;
    const _Float16* row = reinterpret_cast<const _Float16*>(logits) + (int64_t)m * ls;
    const int chunks = N >> 3;

    // Pass 1: maximum and NaN flag. A clamped (repeated) chunk changes neither.
    half2v mx = {(_Float16)(-__builtin_huge_valf()), (_Float16)(-__builtin_huge_valf())};
    uint32_t nan = 0;
    for_row_chunks(row, chunks, tid, [&](int, const uint4& v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mx = __builtin_elementwise_max(mx, __builtin_bit_cast(half2v, w[j]));
            nan |= nan_bits(w[j]);
        }
    });
    float best = fmaxf((float)mx[0], (float)mx[1]);
    for (int n = chunks * 8 + tid; n < N; n += kArgThreads) {
        const uint16_t bits = logits[(int64_t)m * ls + n];
        nan |= nan_bits(bits);
        best = fmaxf(best, (float)row[n]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = fmaxf(best, __shfl_xor(best, o));
    const bool wave_nan = __builtin_amdgcn_ballot_w64(nan != 0) != 0;
    if ((tid & 63) == 0) {
        s_max[tid >> 6] = best;
        s_nan[tid >> 6] = wave_nan;
    }
    __syncthreads();
    bool any_nan = false;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
        best = fmaxf(best, s_max[w]);
        any_nan |= s_nan[w] != 0;
    }
    const _Float16 bh = (_Float16)best;  // exact: the maximum of fp16 values

    // Pass 2: first matching index of this thread (chunks are visited in index order).
    int first = 0x7fffffff;
    auto match = [&](uint32_t w) -> uint32_t {  // 2-bit mask for the two halves of w
        if (any_nan) {
            const uint32_t nb = nan_bits(w);
            return (nb >> 15 & 1u) | (nb >> 30 & 2u);
        }
        const half2v h = __builtin_bit_cast(half2v, w);
        return (uint32_t)(h[0] == bh) | ((uint32_t)(h[1] == bh) << 1);
    };
    // The second read of the row hits L2; keeping the first read's 64 VGPRs live across
    // the block reduction instead measured slower (15.8 vs 10.9 us at 32 x 128256).
    for_row_chunks(row, chunks, tid, [&](int c, const uint4& v) {
        const uint32_t mask = match(v.x) | match(v.y) << 2 | match(v.z) << 4 | match(v.w) << 6;
        if (c < chunks && mask != 0 && first == 0x7fffffff) first = c * 8 + __builtin_ctz(mask);
    });
    for (int n = chunks * 8 + tid; n < N && first == 0x7fffffff; n += kArgThreads)
        if (match(logits[(int64_t)m * ls + n]) & 1u) first = n;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) first = min(first, __shfl_xor(first, o));
    if ((tid & 63) == 0) s_idx[tid >> 6] = first;
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 1; w < kW; ++w) first = min(first, s_idx[w]);
        out[m] = first;
        if (seq_lens) seq_lens[m] += 1;
    }
}

inline bool a16(const void* p) { return aligned(p, 16); }

}  // namespace glue
}  // namespace mx

using namespace mx;

extern "C" int mx_kv_append(const uint16_t* k_new, const uint16_t* v_new, int64_t new_sb, int64_t new_sh,
                            int64_t new_st, int32_t B, int32_t T, int32_t Hkv, int32_t D, const int32_t* block_tables,
                            int64_t bt_sb, int32_t max_blocks, const int32_t* start_pos, uint16_t* k_pool,
                            uint16_t* v_pool, int64_t kv_sblk, int64_t kv_shead, int32_t block_size,
                            int32_t num_pool_blocks, int32_t* err, uint8_t* used_blocks, void* stream) {
    clear_error();
    if (B < 0 || T < 0) return fail(MX_ERR_INVALID, "mx_kv_append: B and T must be >= 0 (B=%d T=%d)", B, T);
    if (B == 0 || T == 0) return MX_OK;
    if (!k_new || !v_new || !block_tables || !start_pos || !k_pool || !v_pool)
        return fail(MX_ERR_NULL, "mx_kv_append: null pointer");
    if (Hkv <= 0 || D <= 0 || D % 8 || block_size <= 0 || max_blocks <= 0 || num_pool_blocks <= 0)
        return fail(MX_ERR_INVALID, "mx_kv_append: need Hkv, max_blocks, block_size, pool > 0 and D %% 8 == 0 "
                                    "(Hkv=%d D=%d bs=%d max_blocks=%d pool=%d)", Hkv, D, block_size, max_blocks,
                    num_pool_blocks);
    if (new_sb % 8 || new_sh % 8 || new_st % 8 || kv_sblk % 8 || kv_shead % 8 || !glue::a16(k_new) ||
        !glue::a16(v_new) || !glue::a16(k_pool) || !glue::a16(v_pool))
        return fail(MX_ERR_ALIGNMENT, "mx_kv_append: states and pool need 16-byte aligned rows");
    glue::AppendParams p{k_new, v_new, new_sb, new_sh, new_st, T, Hkv, D, block_tables, bt_sb, max_blocks,
                         start_pos, k_pool, v_pool, kv_sblk, kv_shead, block_size, num_pool_blocks, err,
                         used_blocks};
    const int64_t total = (int64_t)B * T * Hkv * (D / 8);
    hipLaunchKernelGGL(glue::kv_append_kernel, dim3((unsigned)ceil_div(total, glue::kThreads)), dim3(glue::kThreads),
                       0, as_stream(stream), p, total);
    return check_launch("mx_kv_append");
}

static int rope_append_common(const char* what, glue::RopeAppendParams& p, int32_t B, void* stream) {
    if (B < 0) return fail(MX_ERR_INVALID, "%s: B must be >= 0", what);
    if (B == 0) return MX_OK;
    if (!p.rope || !p.positions || !p.q_out || !p.k_pool || !p.v_pool || !p.bt)
        return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (p.Hq <= 0 || p.Hkv <= 0 || p.D <= 0 || p.D % 8 || p.max_pos <= 0 || p.bs <= 0 || p.max_blocks <= 0 ||
        p.num_pool_blocks <= 0)
        return fail(MX_ERR_INVALID, "%s: need positive sizes and D %% 8 == 0 (Hq=%d Hkv=%d D=%d)", what, p.Hq, p.Hkv,
                    p.D);
    if (p.q_stride % 8 || p.sblk % 8 || p.shead % 8 || !glue::a16(p.q_out) || !glue::a16(p.k_pool) ||
        !glue::a16(p.v_pool) || !aligned(p.rope, 8))
        return fail(MX_ERR_ALIGNMENT, "%s: rows need 16-byte alignment", what);
    if (p.q_stride < (int64_t)p.Hq * p.D) return fail(MX_ERR_INVALID, "%s: q row stride shorter than the row", what);
    const int64_t total = (int64_t)B * (p.Hq + 2 * p.Hkv) * (p.D / 8);
    const dim3 grid((unsigned)ceil_div(total, glue::kThreads)), block(glue::kThreads);
    hipStream_t st = as_stream(stream);
    if (!p.part) hipLaunchKernelGGL(glue::qkv_rope_append_kernel<-1>, grid, block, 0, st, p, total);
    else if (p.splits == 2) hipLaunchKernelGGL(glue::qkv_rope_append_kernel<2>, grid, block, 0, st, p, total);
    else if (p.splits == 4) hipLaunchKernelGGL(glue::qkv_rope_append_kernel<4>, grid, block, 0, st, p, total);
    else if (p.splits == 8) hipLaunchKernelGGL(glue::qkv_rope_append_kernel<8>, grid, block, 0, st, p, total);
    else if (p.splits == 16) hipLaunchKernelGGL(glue::qkv_rope_append_kernel<16>, grid, block, 0, st, p, total);
    else hipLaunchKernelGGL(glue::qkv_rope_append_kernel<0>, grid, block, 0, st, p, total);
    return check_launch(what);
}

extern "C" int mx_qkv_rope_append(const uint16_t* qkv, int64_t qkv_stride, int32_t B, int32_t Hq, int32_t Hkv,
                                  int32_t D, const float* rope, int32_t max_pos, const int32_t* positions,
                                  uint16_t* q_out, int64_t q_stride, uint16_t* k_pool, uint16_t* v_pool,
                                  int64_t kv_sblk, int64_t kv_shead, const int32_t* block_tables, int64_t bt_sb,
                                  int32_t max_blocks, int32_t block_size, int32_t num_pool_blocks, int32_t* err,
                                  int32_t* lens_out, uint8_t* used_blocks, void* stream) {
    clear_error();
    if (B > 0 && !qkv) return fail(MX_ERR_NULL, "mx_qkv_rope_append: null pointer");
    if (B > 0 && (qkv_stride % 8 || !glue::a16(qkv)))
        return fail(MX_ERR_ALIGNMENT, "mx_qkv_rope_append: rows need 16-byte alignment");
    if (B > 0 && qkv_stride < (int64_t)(Hq + 2 * Hkv) * D)
        return fail(MX_ERR_INVALID, "mx_qkv_rope_append: row strides shorter than the rows");
    glue::RopeAppendParams p{qkv, qkv_stride, nullptr, 0, 0, nullptr, Hq, Hkv, D,
                             reinterpret_cast<const float2*>(rope), max_pos, positions, q_out, q_stride, k_pool,
                             v_pool, kv_sblk, kv_shead, block_tables, bt_sb, max_blocks, block_size, num_pool_blocks,
                             err, lens_out, used_blocks};
    return rope_append_common("mx_qkv_rope_append", p, B, stream);
}

extern "C" int mx_qkv_rope_append_splits(const float* partials, int32_t splits, const uint16_t* bias, int32_t B,
                                         int32_t Hq, int32_t Hkv, int32_t D, const float* rope, int32_t max_pos,
                                         const int32_t* positions, uint16_t* q_out, int64_t q_stride,
                                         uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk, int64_t kv_shead,
                                         const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                         int32_t block_size, int32_t num_pool_blocks, int32_t* err,
                                         int32_t* lens_out, uint8_t* used_blocks, void* stream) {
    clear_error();
    if (B > 0 && !partials) return fail(MX_ERR_NULL, "mx_qkv_rope_append_splits: null pointer");
    if (splits < 1) return fail(MX_ERR_INVALID, "mx_qkv_rope_append_splits: splits must be >= 1");
    // The V heads' bias is read 8 halves (16 bytes) at a time, next to 16-byte partial loads.
    if (B > 0 && (!glue::a16(partials) || (bias && !glue::a16(bias))))
        return fail(MX_ERR_ALIGNMENT, "mx_qkv_rope_append_splits: partials and bias need 16-byte alignment");
    const int64_t width = (int64_t)(Hq + 2 * Hkv) * D;
    glue::RopeAppendParams p{nullptr, width, partials, splits, (int64_t)B * width, bias, Hq, Hkv, D,
                             reinterpret_cast<const float2*>(rope), max_pos, positions, q_out, q_stride, k_pool,
                             v_pool, kv_sblk, kv_shead, block_tables, bt_sb, max_blocks, block_size, num_pool_blocks,
                             err, lens_out, used_blocks};
    return rope_append_common("mx_qkv_rope_append_splits", p, B, stream);
}

static int add_rmsnorm_common(const char* what, glue::NormParams& p, int32_t M, void* stream) {
    if (M < 0) return fail(MX_ERR_INVALID, "%s: M must be >= 0", what);
    if (M == 0) return MX_OK;
    if (!p.w || !p.out) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (p.H <= 0 || p.H % 8 || p.H > glue::kNormThreads * 8 * glue::kNormMaxChunks)
        return fail(MX_ERR_INVALID, "%s: need H %% 8 == 0 and H <= %d (H=%d)", what,
                    glue::kNormThreads * 8 * glue::kNormMaxChunks, p.H);
    if (p.os % 8 || (p.res && p.rs % 8) || (p.res_out && p.ros % 8) || !glue::a16(p.w) || !glue::a16(p.out) ||
        (p.res && !glue::a16(p.res)) || (p.res_out && !glue::a16(p.res_out)))
        return fail(MX_ERR_ALIGNMENT, "%s: rows need 16-byte alignment", what);
    const dim3 grid(M), block(glue::kNormThreads);
    hipStream_t st = as_stream(stream);
    if (!p.part) hipLaunchKernelGGL(glue::add_rmsnorm_kernel<-1>, grid, block, 0, st, p);
    else if (p.splits == 2) hipLaunchKernelGGL(glue::add_rmsnorm_kernel<2>, grid, block, 0, st, p);
    else if (p.splits == 4) hipLaunchKernelGGL(glue::add_rmsnorm_kernel<4>, grid, block, 0, st, p);
    else if (p.splits == 8) hipLaunchKernelGGL(glue::add_rmsnorm_kernel<8>, grid, block, 0, st, p);
    else if (p.splits == 16) hipLaunchKernelGGL(glue::add_rmsnorm_kernel<16>, grid, block, 0, st, p);
    else hipLaunchKernelGGL(glue::add_rmsnorm_kernel<0>, grid, block, 0, st, p);
    return check_launch(what);
}

extern "C" int mx_add_rmsnorm(const uint16_t* x, int64_t x_stride, const int64_t* x_rows, int64_t x_count,
                              const uint16_t* residual, int64_t r_stride, const uint16_t* weight, int32_t M, int32_t H, float eps,
                              uint16_t* out, int64_t out_stride, uint16_t* residual_out, int64_t ro_stride,
                              void* stream) {
    clear_error();
    if (M > 0 && !x) return fail(MX_ERR_NULL, "mx_add_rmsnorm: null pointer");
    if (M > 0 && (x_stride % 8 || !glue::a16(x)))
        return fail(MX_ERR_ALIGNMENT, "mx_add_rmsnorm: rows need 16-byte alignment");
    if (x_rows && x_count < 1) return fail(MX_ERR_INVALID, "mx_add_rmsnorm: a gather needs x_count >= 1");
    glue::NormParams p{x, x_stride, x_rows, x_rows ? x_count : (int64_t)M, nullptr, 0, 0, nullptr, residual,
                       r_stride, weight, H, eps, out, out_stride, residual_out, ro_stride};
    return add_rmsnorm_common("mx_add_rmsnorm", p, M, stream);
}

extern "C" int mx_add_rmsnorm_splits(const float* partials, int32_t splits, const uint16_t* bias,
                                     const uint16_t* residual, int64_t r_stride, const uint16_t* weight, int32_t M,
                                     int32_t H, float eps, uint16_t* out, int64_t out_stride,
                                     uint16_t* residual_out, int64_t ro_stride, void* stream) {
    clear_error();
    if (M > 0 && !partials) return fail(MX_ERR_NULL, "mx_add_rmsnorm_splits: null pointer");
    if (splits < 1) return fail(MX_ERR_INVALID, "mx_add_rmsnorm_splits: splits must be >= 1");
    if (M > 0 && (!glue::a16(partials) || (bias && !glue::a16(bias))))
        return fail(MX_ERR_ALIGNMENT, "mx_add_rmsnorm_splits: partials need 16-byte alignment");
    glue::NormParams p{nullptr, H, nullptr, 0, partials, splits, (int64_t)M * H, bias, residual, r_stride, weight, H,
                       eps, out, out_stride, residual_out, ro_stride};
    return add_rmsnorm_common("mx_add_rmsnorm_splits", p, M, stream);
}

extern "C" int mx_silu_mul(const uint16_t* gate_up, int64_t gu_stride, int32_t M, int32_t I, uint16_t* out,
                           int64_t out_stride, void* stream) {
    clear_error();
    if (M < 0) return fail(MX_ERR_INVALID, "mx_silu_mul: M must be >= 0");
    if (M == 0) return MX_OK;
    if (!gate_up || !out) return fail(MX_ERR_NULL, "mx_silu_mul: null pointer");
    if (I <= 0 || I % 8) return fail(MX_ERR_INVALID, "mx_silu_mul: need I %% 8 == 0 (I=%d)", I);
    if (gu_stride % 8 || out_stride % 8 || !glue::a16(gate_up) || !glue::a16(out))
        return fail(MX_ERR_ALIGNMENT, "mx_silu_mul: rows need 16-byte alignment");
    if (gu_stride < 2 * (int64_t)I) return fail(MX_ERR_INVALID, "mx_silu_mul: gate_up row stride < 2*I");
    const int64_t total = (int64_t)M * (I / 8);
    hipLaunchKernelGGL(glue::silu_mul_kernel, dim3((unsigned)ceil_div(total, glue::kThreads)), dim3(glue::kThreads),
                       0, as_stream(stream), gate_up, gu_stride, I, out, out_stride, total);
    return check_launch("mx_silu_mul");
}

extern "C" int mx_swiglu_interleaved(const uint16_t* gate_up, int64_t gu_stride, const float* partials,
                                     int32_t splits, const uint16_t* bias, int32_t M, int32_t I, uint16_t* out,
                                     int64_t out_stride, void* stream) {
    clear_error();
    if (M < 0) return fail(MX_ERR_INVALID, "mx_swiglu_interleaved: M must be >= 0");
    if (M == 0) return MX_OK;
    if (!out || (!gate_up) == (!partials))
        return fail(MX_ERR_NULL, "mx_swiglu_interleaved: need out and exactly one of gate_up / partials");
    if (I <= 0 || I % 8) return fail(MX_ERR_INVALID, "mx_swiglu_interleaved: need I %% 8 == 0 (I=%d)", I);
    if (out_stride < I || out_stride % 8 || !glue::a16(out))
        return fail(MX_ERR_ALIGNMENT, "mx_swiglu_interleaved: output rows must be 16-byte aligned and cover I");
    if (gate_up && (gu_stride < 2 * (int64_t)I || gu_stride % 8 || !glue::a16(gate_up)))
        return fail(MX_ERR_ALIGNMENT, "mx_swiglu_interleaved: gate_up rows must be 16-byte aligned and cover 2I");
    if (partials && (splits < 1 || !glue::a16(partials) || (bias && !glue::a16(bias))))
        return fail(MX_ERR_INVALID, "mx_swiglu_interleaved: need splits >= 1 and 16-byte aligned partials and bias");
    const int64_t total = (int64_t)M * (I / 8);
    const dim3 grid((unsigned)ceil_div(total, glue::kThreads)), block(glue::kThreads);
    hipStream_t st = as_stream(stream);
    if (gate_up) hipLaunchKernelGGL(glue::swiglu_interleaved_kernel<-1>, grid, block, 0, st, gate_up, gu_stride,
                                    nullptr, 0, nullptr, I, out, out_stride, total);
    else if (splits == 2) hipLaunchKernelGGL(glue::swiglu_interleaved_kernel<2>, grid, block, 0, st, nullptr, 0,
                                             partials, splits, bias, I, out, out_stride, total);
    else if (splits == 4) hipLaunchKernelGGL(glue::swiglu_interleaved_kernel<4>, grid, block, 0, st, nullptr, 0,
                                             partials, splits, bias, I, out, out_stride, total);
    else if (splits == 8) hipLaunchKernelGGL(glue::swiglu_interleaved_kernel<8>, grid, block, 0, st, nullptr, 0,
                                             partials, splits, bias, I, out, out_stride, total);
    else hipLaunchKernelGGL(glue::swiglu_interleaved_kernel<0>, grid, block, 0, st, nullptr, 0, partials, splits,
                            bias, I, out, out_stride, total);
    return check_launch("mx_swiglu_interleaved");
}

extern "C" int mx_argmax_rows(const uint16_t* logits, int64_t stride, int32_t M, int32_t N, int64_t* out,
                              int32_t* seq_lens, void* stream) {
    clear_error();
    if (M < 0 || N <= 0) return fail(MX_ERR_INVALID, "mx_argmax_rows: need M >= 0 and N > 0");
    if (M == 0) return MX_OK;
    if (!logits || !out) return fail(MX_ERR_NULL, "mx_argmax_rows: null pointer");
    if (stride < N || stride % 8 || !glue::a16(logits))
        return fail(MX_ERR_ALIGNMENT, "mx_argmax_rows: rows must be 16-byte aligned and cover N");
    hipLaunchKernelGGL(glue::argmax_kernel, dim3(M), dim3(glue::kArgThreads), 0, as_stream(stream), logits, stride, N,
                       out, seq_lens);
    return check_launch("mx_argmax_rows");
}

extern "C" size_t mx_argmax_workspace_bytes(int32_t M, int32_t N) {
    if (M <= 0 || N <= 0) return 0;
    return (size_t)M * (size_t)ceil_div((int64_t)N, glue::kArgChunk) * sizeof(uint64_t);
}

extern "C" int mx_argmax_rows_split(const uint16_t* logits, int64_t stride, int32_t M, int32_t N, int64_t* out,
                                    int32_t* seq_lens, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    const char* what = "mx_argmax_rows_split";
    if (M < 0 || N <= 0) return fail(MX_ERR_INVALID, "%s: need M >= 0 and N > 0", what);
    if (M == 0) return MX_OK;
    if (M > 65535) return fail(MX_ERR_UNSUPPORTED, "%s: M > 65535", what);
    if (!logits || !out || !workspace) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (stride < N || stride % 8 || !glue::a16(logits))
        return fail(MX_ERR_ALIGNMENT, "%s: rows must be 16-byte aligned and cover N", what);
    if (reinterpret_cast<uintptr_t>(workspace) % 8) return fail(MX_ERR_ALIGNMENT, "%s: workspace alignment", what);
    const size_t need = mx_argmax_workspace_bytes(M, N);
    if (workspace_bytes < need)
        return fail(MX_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", what, need, workspace_bytes);
    const int nchunks = (int)ceil_div((int64_t)N, glue::kArgChunk);
    uint64_t* keys = static_cast<uint64_t*>(workspace);
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(glue::argmax_chunk_kernel, dim3(nchunks, M), dim3(glue::kArgChunkThreads), 0, st, logits, stride,
                       N, keys, nchunks);
    hipLaunchKernelGGL(glue::argmax_keys_kernel, dim3(M), dim3(64), 0, st, keys, nchunks, out, seq_lens);
    return check_launch(what);
}
