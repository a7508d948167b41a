// Fused QKV projection + rotate-half RoPE + KV append for the decode step (gfx950).
//
// The decode step's first two kernels per layer, the int8 QKV projection (split-K
// partials) and mx_qkv_rope_append_splits, in one launch. They replace the HF q/k/v
// projections, apply_rotary_pos_emb and BlockPagedBatchLayer.update's K/V write
// (transformers, reached from runtime/phase2/worker_server.py:771-775;
// runtime/phase2/paged_kv_cache.py:121-157).
//
// A workgroup owns the n-tile pair (t, t + D/32) of one head: n-tile t holds dims
// 16 j + [0, 16) of the head and its partner the dims D/2 higher, so every rotate-half
// pair (i, i + D/2) lands in one workgroup and one lane position. Its 8 waves walk the
// 8 k ranges w K / 8 .. (w + 1) K / 8 that mx_w8a16_linear_partials uses for this shape
// at M <= 32, with the same MFMA sequence, so each wave's accumulator equals that
// split's partial before scaling. The epilogue sums the scaled accumulators in LDS,
// bias first and ranges in order, rounds to fp16, rotates with the position's (cos, sin)
// and writes q, k and v as mx_qkv_rope_append_splits does: the results are bit for bit
// those of the two-launch path, without the 6 MB of partials between them.
#include "common.h"
#include "glue_common.h"
#include "w8a16_tiles.h"

namespace mx {
namespace qkvrope {

using w8a16::dequant8;
using w8a16::h2f;
using w8a16::kTileK;
using w8a16::kTileN;

constexpr int kWaves = 8;  // k ranges per workgroup (the split count of the two-launch path)
constexpr int kDepth = 8;       // k-tiles of loads in flight per wave: a whole range at K = 4096
constexpr int kShortDepth = 4;  // ranges of at most this many k-tiles (K <= 2048) with one m-tile
constexpr int kMaxRows = 32;

struct Params {
    const uint16_t* x;
    int64_t xs;
    int M, KT, NT;
    const uint8_t* w;
    const uint16_t* scale;
    const uint16_t* bias;  // NULL: none
    int Hq, Hkv;
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
    int32_t* lens_out;  // optional: lens_out[m] = positions[m] + 1
    uint8_t* used;      // optional [num_pool_blocks] map: 1 where a token was written
};

template <int MT, int D>
__global__ __launch_bounds__(kWaves * 64) void qkv_rope_kernel(Params p) {
    constexpr int HALF = D / (2 * kTileN);  // n-tile pairs per head
    __shared__ float4v red[kWaves][2][MT][64];
    const int pp = blockIdx.x;
    const int head = pp / HALF, jt = pp - head * HALF;
    const int nt0 = head * 2 * HALF + jt, nt1 = nt0 + HALF;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int kt_lo = (int)((int64_t)wave * p.KT / kWaves);
    const int nj = (int)((int64_t)(wave + 1) * p.KT / kWaves) - kt_lo;

    // Positions of the epilogue thread's rows, fetched now so they arrive under the loop.
    const bool epi = tid < MT * 64;
    int pos[4] = {0, 0, 0, 0};
    if (epi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = (tid >> 6) * 16 + 4 * g + i;
            if (m < p.M) pos[i] = p.positions[m];
        }
    }

    // Main loop: the n-tile pair over this wave's k range. x fragments come straight from
    // global memory (L2): lane (r, g) of m-tile mt reads row 16 mt + r, columns
    // 64 kt + 16 g + [0, 16), which are the A operands the split GEMM takes from LDS.
    const uint4* wb = reinterpret_cast<const uint4*>(p.w);
    int xoff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + r;
        xoff[mt] = (int)((row < p.M ? row : p.M - 1) * p.xs) + 16 * g;
    }
    const _Float16* xb = reinterpret_cast<const _Float16*>(p.x);
    struct St {
        uint4 w[2];
        uint4 x[MT][2];
    };
    auto load = [&](int j, St& st) {
        const int kt = kt_lo + (j < nj ? j : nj - 1);
        st.w[0] = w8a16::load_wtile(wb + ((int64_t)kt * p.NT + nt0) * 64 + lane);
        st.w[1] = w8a16::load_wtile(wb + ((int64_t)kt * p.NT + nt1) * 64 + lane);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const uint4* src = reinterpret_cast<const uint4*>(xb + xoff[mt] + kt * kTileK);
            st.x[mt][0] = src[0];
            st.x[mt][1] = src[1];
        }
    };
    float4v acc[2][MT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const St& st) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const half8v b0 = dequant8(st.w[t].x, st.w[t].y);
            const half8v b1 = dequant8(st.w[t].z, st.w[t].w);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, st.x[mt][0]), b0,
                                                                    acc[t][mt], 0, 0, 0);
                acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, st.x[mt][1]), b1,
                                                                    acc[t][mt], 0, 0, 0);
            }
        }
    };
    // Rotation factors, pool slots, scales and bias of the epilogue thread's rows. With one m-tile
    // and a short k range (at most kShortDepth k-tiles, all in flight at once) their loads are
    // issued right after the pipeline's loads (the positions, loaded first, have arrived by
    // then), so they overlap the main loop instead of adding a round trip after it: qkv
    // 8.2 -> 6.5 us on the Qwen2-0.5B shape at 16 rows. Otherwise they follow the loop, still
    // ahead of the workgroup's final barrier: held through the 8-deep loop the early values cost
    // registers (two m-tiles: 236 -> 256 VGPRs, 12.6 -> 13.3 us at 32 rows; one m-tile at
    // K = 4096 with a 4-deep loop instead: 9.3-10.1 -> 10.4 us at 16 rows).
    const int c = jt * kTileN + r;  // dim of the pair's first element within the head
    const int n0 = nt0 * kTileN + r, n1 = nt1 * kTileN + r;
    float2 cs[4];
    int64_t dst[4];
    float sc0 = 0.0f, sc1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
    auto epilogue_inputs = [&]() {
        sc0 = h2f(p.scale, n0);
        sc1 = h2f(p.scale, n1);
        if (p.bias) {
            b0 = h2f(p.bias, n0);
            b1 = h2f(p.bias, n1);
        }
        if (!epi) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = (tid >> 6) * 16 + 4 * g + i;
            const int ps = pos[i];
            const bool live = m < p.M && ps >= 0 && ps < p.max_pos;
            cs[i] = live && head < p.Hq + p.Hkv ? p.rope[(int64_t)ps * (D / 2) + c] : float2{0.0f, 0.0f};
            dst[i] = -1;
            if (live && head >= p.Hq) {
                const int kvh = head < p.Hq + p.Hkv ? head - p.Hq : head - p.Hq - p.Hkv;
                dst[i] = glue::slot_offset(p.bt, p.bt_sb, p.max_blocks, m, ps, p.bs, p.num_pool_blocks, p.sblk,
                                           p.shead, kvh, D);
            }
        }
    };
    if (MT == 1 && nj > 0 && nj <= kShortDepth) {
        // The range's tiles only (no clamped repeats of the last one), then the unrolled compute:
        // Qwen2-0.5B shape at 16 rows 6.5 -> 5.24 us on MI355X. The same form for the 8-deep ranges
        // (Llama-3-8B shape, 32 rows) measured slower (12.5 -> 13.15 us) and is not used there.
        St st[kShortDepth];
#pragma unroll
        for (int j = 0; j < kShortDepth; ++j)
            if (j < nj) load(j, st[j]);
        epilogue_inputs();
#pragma unroll
        for (int j = 0; j < kShortDepth; ++j)
            if (j < nj) compute(st[j]);
    } else {
        if (nj > 0) {
            St st[kDepth];
            PIPELINE_BODY(kDepth, nj, st, load, compute(st[s]))
        }
        epilogue_inputs();
    }

    // Scaled accumulators (the split partials) to LDS; acc[t][mt][i] is row
    // 16 mt + 4 g + i, column 16 nt + r of tile t.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        float4v v0, v1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v0[i] = pin_f32(acc[0][mt][i] * sc0);
            v1[i] = pin_f32(acc[1][mt][i] * sc1);
        }
        red[wave][0][mt][lane] = v0;
        red[wave][1][mt][lane] = v1;
    }
    __syncthreads();
    if (!epi) return;

    const int mt = tid >> 6;
    float s0[4], s1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s0[i] = b0;
        s1[i] = b1;
    }
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const float4v v0 = red[w][0][mt][lane], v1 = red[w][1][mt][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0[i] += v0[i];
            s1[i] += v1[i];
        }
    }
    const bool flag_lane = r == 0 && jt == 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = mt * 16 + 4 * g + i;
        if (m >= p.M) continue;
        const _Float16 x1 = (_Float16)pin_f32(s0[i]), x2 = (_Float16)pin_f32(s1[i]);
        const int ps = pos[i];
        const bool pos_ok = ps >= 0 && ps < p.max_pos;
        if (pp == 0 && r == 0 && p.lens_out) p.lens_out[m] = ps + 1;
        if (head < p.Hq + p.Hkv) {
            half2v o = {(_Float16)0.0f, (_Float16)0.0f};
            if (pos_ok) o = glue::rope_rotate(x1, x2, cs[i]);
            else if (p.err && flag_lane) atomicOr(p.err, 2);
            if (head < p.Hq) {
                _Float16* q = reinterpret_cast<_Float16*>(p.q_out) + (int64_t)m * p.q_stride + (int64_t)head * D + c;
                q[0] = o[0];
                q[D / 2] = o[1];
                continue;
            }
            if (!pos_ok) continue;
            if (dst[i] < 0) {
                if (p.err && flag_lane) atomicOr(p.err, 1);
                continue;
            }
            _Float16* k = reinterpret_cast<_Float16*>(p.k_pool) + dst[i] + c;
            k[0] = o[0];
            k[D / 2] = o[1];
            if (p.used && flag_lane && head == p.Hq) p.used[p.bt[(int64_t)m * p.bt_sb + ps / p.bs]] = 1;
        } else {
            if (dst[i] < 0) continue;  // position or slot outside the tables: flagged by the q/k heads
            _Float16* v = reinterpret_cast<_Float16*>(p.v_pool) + dst[i] + c;
            v[0] = x1;
            v[D / 2] = x2;
        }
    }
}

template <int D>
static void launch(const Params& p, hipStream_t st) {
    const dim3 grid(p.NT / 2), block(kWaves * 64);
    if (p.M <= 16) hipLaunchKernelGGL((qkv_rope_kernel<1, D>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((qkv_rope_kernel<2, D>), grid, block, 0, st, p);
}

}  // namespace qkvrope
}  // namespace mx

using namespace mx;

extern "C" int mx_w8a16_qkv_rope_append(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride,
                                        const uint8_t* packed, const uint16_t* scale, const uint16_t* bias,
                                        int32_t Hq, int32_t Hkv, int32_t D, const float* rope, int32_t max_pos,
                                        const int32_t* positions, uint16_t* q_out, int64_t q_stride,
                                        uint16_t* k_pool, uint16_t* v_pool, int64_t kv_sblk, int64_t kv_shead,
                                        const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                        int32_t block_size, int32_t num_pool_blocks, int32_t* err, int32_t* lens_out,
                                        uint8_t* used_blocks, void* stream) {
    const char* what = "mx_w8a16_qkv_rope_append";
    clear_error();
    if (M < 0) return fail(MX_ERR_INVALID, "%s: M must be >= 0", what);
    if (M == 0) return MX_OK;
    if (M > qkvrope::kMaxRows) return fail(MX_ERR_UNSUPPORTED, "%s: M = %lld > %d rows", what, (long long)M, qkvrope::kMaxRows);
    if (D != 64 && D != 128) return fail(MX_ERR_UNSUPPORTED, "%s: head_dim %d unsupported (64 or 128)", what, D);
    if (!x || !packed || !scale || !rope || !positions || !q_out || !k_pool || !v_pool || !block_tables)
        return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (Hq <= 0 || Hkv <= 0 || max_pos <= 0 || block_size <= 0 || max_blocks <= 0 || num_pool_blocks <= 0)
        return fail(MX_ERR_INVALID, "%s: need positive sizes (Hq=%d Hkv=%d)", what, Hq, Hkv);
    if (K <= 0 || K % w8a16::kTileK) return fail(MX_ERR_INVALID, "%s: K must be a positive multiple of 64", what);
    if (x_stride < K || x_stride % 8 || !aligned(x, 16) || !aligned(packed, 16) || !aligned(scale, 2) ||
        (bias && !aligned(bias, 2)))
        return fail(MX_ERR_ALIGNMENT, "%s: x rows need 16-byte alignment and stride >= K", what);
    if (q_stride < (int64_t)Hq * D || kv_sblk % 8 || kv_shead % 8 || !aligned(rope, 8))
        return fail(MX_ERR_INVALID, "%s: bad q stride or pool strides", what);
    qkvrope::Params p{};
    p.x = x;
    p.xs = x_stride;
    p.M = (int)M;
    p.KT = (int)(K / w8a16::kTileK);
    p.NT = (Hq + 2 * Hkv) * D / w8a16::kTileN;
    p.w = packed;
    p.scale = scale;
    p.bias = bias;
    p.Hq = Hq;
    p.Hkv = Hkv;
    p.rope = reinterpret_cast<const float2*>(rope);
    p.max_pos = max_pos;
    p.positions = positions;
    p.q_out = q_out;
    p.q_stride = q_stride;
    p.k_pool = k_pool;
    p.v_pool = v_pool;
    p.sblk = kv_sblk;
    p.shead = kv_shead;
    p.bt = block_tables;
    p.bt_sb = bt_sb;
    p.max_blocks = max_blocks;
    p.bs = block_size;
    p.num_pool_blocks = num_pool_blocks;
    p.err = err;
    p.lens_out = lens_out;
    p.used = used_blocks;
    hipStream_t st = as_stream(stream);
    if (D == 128) qkvrope::launch<128>(p, st);
    else qkvrope::launch<64>(p, st);
    return check_launch(what);
}
