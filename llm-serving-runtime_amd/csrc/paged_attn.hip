// Paged-attention decode for gfx950.
//
// Replaces paged_attention_decode_batched (runtime/phase2/paged_attention_triton.py:745-775)
// and its Triton kernels: the direct batched kernel (:148-243), the B=1
// split kernel (:245-336), the B=1 direct kernel (:338-412) and the log-sum-exp
// combine (:414-457), for any batch and any mix of context lengths.
//
// Kernel 1 (partial): one workgroup (4 waves) per (token chunk, kv-head,
// sequence). The G = Hq/Hkv query heads of a kv-head share every K/V byte the
// workgroup reads, so K/V are fetched once per kv-head (the reference grid
// (B, Hq) re-reads them G times, :179-181). Chunks are fixed-size runs of
// tokens, so a long row gets more workgroups than a short one (ragged-aware
// split-K, where the reference splits only B=1 rows, :82-87, :537-552).
//
// Per 16-token tile a wave:
//   * loads K rows as the A operand of v_mfma_f32_16x16x32_f16 (16 tokens x
//     32 dims per instruction, one 128-bit load per lane), with the G query
//     heads (zero padded to 16) as the B operand -> scores S[token][head];
//   * runs the online softmax in fp32 on the exp2 scale (scores are
//     pre-multiplied by scale*log2(e); exp2(x*log2 e) == exp(x));
//   * shares p[token][head] and the rescale factor through a per-wave LDS
//     slot and accumulates P.V on the VALU from V rows loaded as contiguous
//     1 KiB runs (lane: 8 dims of RPL-strided tokens), fp32 accumulation.
// A wave keeps two tiles in flight (the next tile's K/V loads are issued
// before the current tile is computed) and reads its block ids for the whole
// chunk with one vector load up front. Waves merge in LDS. A row covered by
// one chunk is written directly; otherwise the chunk's fp32 partial
// (m, l, acc[G][D]) goes to the workspace.
//
// Kernel 2 (combine): one workgroup per (kv-head, sequence) with more than one
// chunk applies the log-sum-exp merge and writes fp16 output. Splitting the
// merge into its own launch keeps kernel 1 free of device-scope fences: on
// gfx950 a release/acquire at agent scope writes back and invalidates the XCD's
// L2, which serialises thousands of workgroups.
#include "common.h"

namespace mx {
namespace pa {

struct Params {
    const _Float16* q;
    int64_t q_sb, q_sh;
    const _Float16* k;
    const _Float16* v;
    int64_t kv_sblk, kv_shead;
    const int32_t* bt;
    int64_t bt_sb;
    int max_blocks;
    const int32_t* seq_lens;
    int Hkv;
    int num_pool_blocks;
    float scale_log2e;
    _Float16* out;
    int64_t o_sb, o_sh;
    float* part_ml;   // [B*Hkv*max_chunks][G][2]  (m, l) on the exp2 scale
    float* part_acc;  // [B*Hkv*max_chunks][G][D]
    int* err;         // error word
    int max_chunks;
    int chunk_tiles;
};

constexpr int kWaves = 4;
constexpr int kTile = 16;  // tokens per MFMA tile
constexpr int kDefaultChunkTokens = 256;
constexpr int kMaxChunkTokens = kWaves * 64 * kTile;  // a wave prefetches at most 64 block ids
constexpr int kMaxChunks = 1024;                      // combine kernel keeps chunk weights in LDS

__device__ __forceinline__ half8v load_half8(const _Float16* p) {
    return __builtin_bit_cast(half8v, *reinterpret_cast<const uint4*>(p));
}

// Number of 16-token chunks of a row, shared by both kernels.
template <int BS>
__device__ __forceinline__ void row_extent(int S, int max_blocks, int chunk_tiles, int& s_eff, int& ntiles,
                                           int& nchunks) {
    int nblk = S > 0 ? (S + BS - 1) / BS : 0;
    if (nblk > max_blocks) nblk = max_blocks;
    s_eff = S < nblk * BS ? S : nblk * BS;
    ntiles = (s_eff + kTile - 1) / kTile;
    nchunks = (ntiles + chunk_tiles - 1) / chunk_tiles;
}

template <int KK, int NL>
struct TileRegs {
    half8v k[KK];
    half8v v[NL];
};

// Pipeline depth from the VGPRs of one tile stage (K and V, 4 per fragment)
// after the G*8 accumulators.
constexpr int pa_depth(int D, int G) {
    const int d = (160 - 8 * G) / (4 * (D / 32 + D / 32));
    return d < 2 ? 2 : (d > 4 ? 4 : d);
}

template <int D, int BS, int G>
__global__ __launch_bounds__(kWaves * 64) void decode_partial_kernel(Params p) {
    constexpr int KK = D / 32;       // MFMA k-steps over the head dim
    constexpr int LPR = D / 8;       // lanes per token row when loading V
    constexpr int RPL = 64 / LPR;    // token rows per V load instruction
    constexpr int NL = kTile / RPL;  // V load instructions per tile
    constexpr int TPB = BS / kTile;  // tiles per KV block
    constexpr int P = pa_depth(D, G);
    const float kNegInf = -__builtin_huge_valf();

    const int chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, r = lane & 15;
    const int h0 = kvh * G;

    int s_eff, ntiles, nchunks;
    row_extent<BS>(p.seq_lens[b], p.max_blocks, p.chunk_tiles, s_eff, ntiles, nchunks);

    _Float16* out_row = p.out + (int64_t)b * p.o_sb + (int64_t)h0 * p.o_sh;
    if (nchunks == 0) {  // empty row: defined as a zero output
        if (chunk == 0) {
            for (int idx = tid; idx < G * D; idx += kWaves * 64)
                out_row[(int64_t)(idx / D) * p.o_sh + idx % D] = (_Float16)0.0f;
        }
        return;
    }
    if (chunk >= nchunks) return;
    const int t_begin = chunk * p.chunk_tiles;
    const int t_end = (t_begin + p.chunk_tiles) < ntiles ? (t_begin + p.chunk_tiles) : ntiles;
    const int t_first = t_begin + wave;
    const int nj = t_first < t_end ? (t_end - t_first + kWaves - 1) / kWaves : 0;  // tiles of this wave

    __shared__ float s_p[kWaves][kTile][17];
    __shared__ float s_alpha[kWaves][16];
    __shared__ float s_m[kWaves][G];
    __shared__ float s_l[kWaves][G];
    __shared__ float s_acc[kWaves][G][D];

    // Block ids of this wave's tiles: lane j holds the id of tile t_first + 4*j;
    // an id outside the pool becomes -1 (tile skipped, error recorded).
    const int32_t* bt_row = p.bt + (int64_t)b * p.bt_sb;
    int my_pb = 0;
    if (lane < nj) {
        my_pb = bt_row[(t_first + kWaves * lane) / TPB];
        if ((unsigned)my_pb >= (unsigned)p.num_pool_blocks) {  // never read outside the pool
            atomicOr(p.err, 1);
            my_pb = -1;
        }
    }

    // B operand: query head r (zero past G), dims 32*kk + 8*g + [0, 8).
    half8v qf[KK];
    if (r < G) {
        const _Float16* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(h0 + r) * p.q_sh + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qf[kk] = load_half8(qp + 32 * kk);
    } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qf[kk] = (_Float16)0.0f;
    }

    float m_run = kNegInf;  // running max of head r (same in all 4 lane groups)
    float l_run = 0.0f;     // partial denominator over this lane's tokens
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    const _Float16* kbase = p.k + (int64_t)kvh * p.kv_shead;
    const _Float16* vbase = p.v + (int64_t)kvh * p.kv_shead;
    const int vrow = lane / LPR, vcol = (lane % LPR) * 8;
    const int koff = r * D + 8 * g;
    const int voff = vrow * D + vcol;

    // Loads are unconditional: past the wave's last tile the index is clamped
    // (an L2 hit) and a skipped block reads block 0; only the compute below is
    // predicated, by wave-uniform flags, so waits count exact stages.
    auto load_tile = [&](int j, TileRegs<KK, NL>& tr) {
        const int jc = j < nj ? j : nj - 1;
        const int pb = __builtin_amdgcn_readlane(my_pb, jc);
        const int t = t_first + kWaves * jc;
        const int64_t base = (int64_t)(pb < 0 ? 0 : pb) * p.kv_sblk + (t % TPB) * kTile * D;
        const _Float16* kt = kbase + base;
        const _Float16* vt = vbase + base;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) tr.k[kk] = load_half8(kt + koff + 32 * kk);
#pragma unroll
        for (int jj = 0; jj < NL; ++jj) tr.v[jj] = load_half8(vt + voff + jj * RPL * D);
    };

    auto compute_tile = [&](int j, const TileRegs<KK, NL>& tr) {
        const int t = t_first + kWaves * j;
        float4v s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(tr.k[kk], qf[kk], s, 0, 0, 0);
        // s[i] = score of token t*16 + 4g + i for head r.
        const int tok0 = t * kTile + 4 * g;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = (tok0 + i < s_eff) ? s[i] * p.scale_log2e : kNegInf;
        const float mx = xor_max_16_32(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        float psum = 0.0f;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float pi = __builtin_amdgcn_exp2f(sc[i] - m_new);
            s_p[wave][4 * g + i][r] = pi;
            psum += pi;
        }
        l_run = l_run * alpha + psum;
        const bool rescale = __builtin_amdgcn_ballot_w64(m_new != m_run) != 0;
        m_run = m_new;
        if (g == 0) s_alpha[wave][r] = alpha;
        __builtin_amdgcn_wave_barrier();
        // P.V on the VALU: this lane owns dims vcol..vcol+7 of tokens jj*RPL + vrow.
        if (rescale) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float a = s_alpha[wave][h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] *= a;
            }
        }
#pragma unroll
        for (int jj = 0; jj < NL; ++jj) {
            const int tok = jj * RPL + vrow;
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float pj = s_p[wave][tok][h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pj, (float)tr.v[jj][e], acc[h][e]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    if (nj > 0) {
        TileRegs<KK, NL> st[P];
#pragma unroll
        for (int s = 0; s < P; ++s) load_tile(s, st[s]);
        for (int j0 = 0; j0 < nj; j0 += P) {
#pragma unroll
            for (int s = 0; s < P; ++s) {
                const int j = j0 + s;
                if (j < nj && __builtin_amdgcn_readlane(my_pb, j) >= 0) compute_tile(j, st[s]);
                load_tile(j + P, st[s]);
            }
        }
    }

    // Wave totals: l over the 4 lane groups, acc over the token groups.
    l_run = xor_sum_16_32(l_run);
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[h][e];
            if (LPR == 8) v = xor8_sum(v);
            acc[h][e] = xor_sum_16_32(v);
        }
    if (g == 0 && r < G) {
        s_m[wave][r] = m_run;
        s_l[wave][r] = l_run;
    }
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) s_acc[wave][h][vcol + e] = acc[h][e];
    }
    __syncthreads();

    const int64_t pslot = ((int64_t)b * p.Hkv + kvh) * p.max_chunks + chunk;
    for (int idx = tid; idx < G * D; idx += kWaves * 64) {
        const int h = idx / D, d = idx % D;
        float mw = s_m[0][h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mw = fmaxf(mw, s_m[w][h]);
        float lw = 0.0f, aw = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float f = exp2f(s_m[w][h] - mw);
            lw += f * s_l[w][h];
            aw += f * s_acc[w][h][d];
        }
        if (nchunks == 1) {
            out_row[(int64_t)h * p.o_sh + d] = (_Float16)(aw / lw);
        } else {
            p.part_acc[(pslot * G + h) * D + d] = aw;
            if (d == 0) {
                p.part_ml[(pslot * G + h) * 2 + 0] = mw;
                p.part_ml[(pslot * G + h) * 2 + 1] = lw;
            }
        }
    }
}

// Log-sum-exp merge of the chunk partials of one (kv-head, sequence).
template <int D, int BS, int G>
__global__ __launch_bounds__(256) void decode_combine_kernel(Params p) {
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x;
    int s_eff, ntiles, nchunks;
    row_extent<BS>(p.seq_lens[b], p.max_blocks, p.chunk_tiles, s_eff, ntiles, nchunks);
    if (nchunks <= 1) return;
    __shared__ float s_w[kMaxChunks][G];
    __shared__ float s_inv_l[G];
    const int64_t base = ((int64_t)b * p.Hkv + kvh) * p.max_chunks;
    if (tid < G) {
        const int h = tid;
        float mg = -__builtin_huge_valf();
        for (int c = 0; c < nchunks; ++c) mg = fmaxf(mg, p.part_ml[((base + c) * G + h) * 2]);
        float lg = 0.0f;
        for (int c = 0; c < nchunks; ++c) {
            const float f = exp2f(p.part_ml[((base + c) * G + h) * 2] - mg);
            s_w[c][h] = f;
            lg += f * p.part_ml[((base + c) * G + h) * 2 + 1];
        }
        s_inv_l[h] = 1.0f / lg;
    }
    __syncthreads();
    _Float16* out_row = p.out + (int64_t)b * p.o_sb + (int64_t)(kvh * G) * p.o_sh;
    for (int idx = tid; idx < G * D; idx += 256) {
        const int h = idx / D, d = idx % D;
        float a = 0.0f;
        for (int c = 0; c < nchunks; ++c) a += s_w[c][h] * p.part_acc[((base + c) * G + h) * D + d];
        out_row[(int64_t)h * p.o_sh + d] = (_Float16)(a * s_inv_l[h]);
    }
}

struct Layout {
    size_t err, ml, acc, total;
    int max_chunks, chunk_tokens;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Default chunk: the largest of 2048/1024/512/256 tokens that still gives about
// one workgroup per CU when rows are, on average, half the table width.
// Larger chunks amortise each workgroup's start-up and the merge; smaller ones
// keep a few long rows spread over the chip. Host-only: no seq_lens read.
static int resolve_chunk_tokens(int chunk_tokens, int B, int Hkv, int max_blocks, int block_size) {
    if (chunk_tokens > 0) return chunk_tokens;
    const int64_t half_row = ((int64_t)max_blocks * block_size + 1) / 2;
    for (int ct = 2048; ct > kDefaultChunkTokens; ct /= 2) {
        if ((int64_t)B * Hkv * ceil_div(half_row, ct) >= 256) return ct;
    }
    return kDefaultChunkTokens;
}

static Layout layout(int B, int Hq, int Hkv, int D, int max_blocks, int block_size, int chunk_tokens) {
    Layout L{};
    L.chunk_tokens = resolve_chunk_tokens(chunk_tokens, B, Hkv, max_blocks, block_size);
    const int64_t max_tokens = (int64_t)max_blocks * block_size;
    L.max_chunks = (int)(max_tokens > 0 ? ceil_div(max_tokens, L.chunk_tokens) : 1);
    const int G = Hkv > 0 ? Hq / Hkv : 0;
    const size_t units = (size_t)B * Hkv;
    L.err = 0;
    L.ml = 256;
    L.acc = L.ml + align256(units * L.max_chunks * G * 2 * sizeof(float));
    L.total = L.acc + align256(units * L.max_chunks * G * D * sizeof(float));
    return L;
}

template <int D, int BS, int G>
static void launch(const Params& prm, int B, hipStream_t st) {
    hipLaunchKernelGGL((decode_partial_kernel<D, BS, G>), dim3(prm.max_chunks, prm.Hkv, B), dim3(kWaves * 64), 0, st,
                       prm);
    if (prm.max_chunks > 1)
        hipLaunchKernelGGL((decode_combine_kernel<D, BS, G>), dim3(prm.Hkv, B), dim3(256), 0, st, prm);
}

template <int D, int BS>
static bool dispatch_g(int G, const Params& prm, int B, hipStream_t st) {
    switch (G) {
        case 1: launch<D, BS, 1>(prm, B, st); return true;
        case 2: launch<D, BS, 2>(prm, B, st); return true;
        case 3: launch<D, BS, 3>(prm, B, st); return true;
        case 4: launch<D, BS, 4>(prm, B, st); return true;
        case 5: launch<D, BS, 5>(prm, B, st); return true;
        case 6: launch<D, BS, 6>(prm, B, st); return true;
        case 7: launch<D, BS, 7>(prm, B, st); return true;
        case 8: launch<D, BS, 8>(prm, B, st); return true;
        default: return false;
    }
}

}  // namespace pa
}  // namespace mx

using namespace mx;

extern "C" size_t mx_paged_attn_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                                int32_t block_size, int32_t chunk_tokens) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_blocks < 0 || block_size <= 0) return 0;
    return pa::layout(B, Hq, Hkv, D, max_blocks, block_size, chunk_tokens).total;
}

extern "C" size_t mx_paged_attn_error_offset(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                             int32_t block_size, int32_t chunk_tokens) {
    return pa::layout(B, Hq, Hkv, D, max_blocks, block_size, chunk_tokens).err;
}

extern "C" int mx_paged_attn_decode(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                                    const uint16_t* v, int64_t kv_sblk, int64_t kv_shead,
                                    const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                    const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                    int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out,
                                    int64_t o_sb, int64_t o_sh, void* workspace, size_t workspace_bytes,
                                    int32_t chunk_tokens, void* stream) {
    if (B < 0) return fail(MX_ERR_INVALID, "mx_paged_attn_decode: B must be >= 0");
    if (B == 0) return MX_OK;
    if (!q || !k || !v || !block_tables || !seq_lens || !out)
        return fail(MX_ERR_NULL, "mx_paged_attn_decode: null pointer");
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
        return fail(MX_ERR_INVALID, "mx_paged_attn_decode: Hq (%d) must be a positive multiple of Hkv (%d)", Hq, Hkv);
    const int G = Hq / Hkv;
    if (G > 8) return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: GQA group %d > 8 unsupported", G);
    if (D != 64 && D != 128) return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: head_dim %d unsupported", D);
    if (block_size != 16 && block_size != 32)
        return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: block_size %d unsupported (16 or 32)", block_size);
    if (max_blocks < 1 || num_pool_blocks < 1)
        return fail(MX_ERR_INVALID, "mx_paged_attn_decode: max_blocks and num_pool_blocks must be >= 1");
    if (B > 65535 || Hkv > 65535) return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: B or Hkv too large");
    const int ct = pa::resolve_chunk_tokens(chunk_tokens, B, Hkv, max_blocks, block_size);
    if (ct % pa::kTile != 0 || ct > pa::kMaxChunkTokens)
        return fail(MX_ERR_INVALID, "mx_paged_attn_decode: chunk_tokens must be a multiple of 16 and <= %d",
                    pa::kMaxChunkTokens);
    if (!aligned(q, 16) || q_sb % 8 || q_sh % 8 || !aligned(k, 16) || !aligned(v, 16) || kv_sblk % 8 ||
        kv_shead % 8 || !aligned(out, 2))
        return fail(MX_ERR_ALIGNMENT, "mx_paged_attn_decode: q/K/V rows must be 16-byte aligned");
    const pa::Layout L = pa::layout(B, Hq, Hkv, D, max_blocks, block_size, ct);
    if (L.max_chunks > pa::kMaxChunks)
        return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: max_blocks*block_size/chunk_tokens exceeds %d chunks",
                    pa::kMaxChunks);
    if (!workspace || workspace_bytes < L.total)
        return fail(MX_ERR_WORKSPACE, "mx_paged_attn_decode: workspace needs %zu bytes, got %zu", L.total,
                    workspace_bytes);
    if (!aligned(workspace, 256)) return fail(MX_ERR_ALIGNMENT, "mx_paged_attn_decode: workspace must be 256-byte aligned");

    char* ws = static_cast<char*>(workspace);
    pa::Params prm{};
    prm.q = reinterpret_cast<const _Float16*>(q);
    prm.q_sb = q_sb;
    prm.q_sh = q_sh;
    prm.k = reinterpret_cast<const _Float16*>(k);
    prm.v = reinterpret_cast<const _Float16*>(v);
    prm.kv_sblk = kv_sblk;
    prm.kv_shead = kv_shead;
    prm.bt = block_tables;
    prm.bt_sb = bt_sb;
    prm.max_blocks = max_blocks;
    prm.seq_lens = seq_lens;
    prm.Hkv = Hkv;
    prm.num_pool_blocks = num_pool_blocks;
    prm.scale_log2e = scale * 1.4426950408889634f;
    prm.out = reinterpret_cast<_Float16*>(out);
    prm.o_sb = o_sb;
    prm.o_sh = o_sh;
    prm.err = reinterpret_cast<int*>(ws + L.err);
    prm.part_ml = reinterpret_cast<float*>(ws + L.ml);
    prm.part_acc = reinterpret_cast<float*>(ws + L.acc);
    prm.max_chunks = L.max_chunks;
    prm.chunk_tiles = ct / pa::kTile;
    hipStream_t st = as_stream(stream);
    bool ok = false;
    if (D == 128 && block_size == 16) ok = pa::dispatch_g<128, 16>(G, prm, B, st);
    else if (D == 128 && block_size == 32) ok = pa::dispatch_g<128, 32>(G, prm, B, st);
    else if (D == 64 && block_size == 16) ok = pa::dispatch_g<64, 16>(G, prm, B, st);
    else ok = pa::dispatch_g<64, 32>(G, prm, B, st);
    if (!ok) return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode: unsupported configuration");
    return check_launch("mx_paged_attn_decode");
}
