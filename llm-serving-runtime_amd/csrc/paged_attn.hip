// Paged-attention decode for gfx950.
//
// Replaces paged_attention_decode_batched (runtime/phase2/paged_attention_triton.py:745-775)
// and its Triton kernels: the direct batched kernel (:148-243), the B=1
// split kernel (:245-336), the B=1 direct kernel (:338-412) and the log-sum-exp
// combine (:414-457), for any batch and any mix of context lengths.
//
// Work decomposition. A segment is one (sequence, kv-head) pair; it holds
// ceil(seq_len / 16) tiles of 16 tokens. The G = Hq/Hkv query heads of a
// kv-head share every K/V byte of the segment, so K/V are read once per
// kv-head (the reference grid (B, Hq) re-reads them G times, :179-181). All
// segments, row-major over (sequence, kv-head), form one sequence of T tiles
// that is cut into W = min(workers, T) equal contiguous ranges, one per wave
// ("worker"): worker w owns tiles [floor(w T / W), floor((w + 1) T / W)), at
// least one. Every wave thus
// streams the same number of K/V bytes whatever the mix of context lengths, so
// the chip drains evenly (fixed per-sequence chunks leave a long tail when
// lengths are ragged, and the reference splits only B=1 rows, :82-87,
// :537-552).
//
// Kernel 1 (split): a wave walks its range; for each segment piece it
//   * loads K rows as the A operand of v_mfma_f32_16x16x32_f16 (16 tokens x
//     32 dims per instruction, one 128-bit load per lane), with the G query
//     heads (zero padded to 16) as the B operand -> scores S[token][head]:
//     lane l holds the scores of tokens 4*(l/16) + i, i < 4, for head l%16;
//   * runs the online softmax in fp32 on the exp2 scale (scores are
//     pre-multiplied by scale*log2(e); exp2(x*log2 e) == exp(x)), moving the
//     reference maximum only when it rises by more than 2^8;
//   * accumulates P.V with v_mfma_f32_16x16x16_f16, contracting over the
//     tile's 16 tokens. Each lane loads V for exactly the four tokens whose
//     probabilities it already holds, at D/16 consecutive dims, so both
//     operands are lane-local: MFMA e takes A[m][k] = V[token k][m*D/16 + e]
//     and B[k][n] = p[token k][head n], and lane l accumulates output dims
//     (4*(l/16) + i)*D/16 + e of head l%16. p enters the product rounded to
//     fp16 (the reference's SDPA fallback also multiplies fp16
//     probabilities into V); the denominator sums the same rounded values;
//   * keeps P tiles of K/V loads in flight and reads the piece's block ids
//     with one vector load (a range never exceeds 64 tiles).
// A piece that is a whole segment is written as fp16 output; otherwise its
// partial, (m, l) in fp32 and its own output acc / l rounded to the element type
// (fp16 or bf16, half the bytes of the fp32 accumulator; the merge weights it by
// l again), goes to the segment's window of U slots: piece k of segment s (the
// k-th worker that cuts it) to slot s*U + k, and pieces k >= U to an overflow
// slot, B*Hkv*U + w (only a worker's first piece can have k >= 1, so one
// overflow slot per worker suffices). The workers holding a segment's first and
// last tile record themselves in seg_w.
//
// Kernel 2 (merge): one workgroup per segment issues the loads of its lengths,
// its worker span and its whole window of U slots at once, applies the
// log-sum-exp merge of the partials and writes fp16 output (zeros for an empty
// row): one memory round trip for a segment of at most U pieces, a second one
// for the overflow slots of longer ones. The merge has a
// launch of its own because handing partials between workgroups inside one
// launch costs more on gfx950 than the launch: an agent-scope release/acquire
// writes back and invalidates the XCD's L2 (measured 2.6x slower at the bench
// shape), and write-through atomic partials with a ticket counter still lost
// (1.3x).
#include <mutex>
#include <type_traits>

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
    int B, Hkv;
    int num_pool_blocks;
    float scale_log2e;
    _Float16* out;
    int64_t o_sb, o_sh;
    float* part_ml;   // [slots][G][2]  (m, l) on the exp2 scale
    _Float16* part_out;  // [slots][G][D]: each piece's output normalised by its own l, element type
    int* seg_w;       // [B*Hkv][2]: workers holding the first and the last tile of a segment
    int* err;         // error word
    int workers;
    int wg_waves;     // waves per workgroup of the split launch (<= kWaves)
    int vg;           // virtual kv-heads per pool head (GQA groups above 8, see kv_virtual_groups)
    int4* plan;       // [workers][65] tile plan: written by a MX_PA_PLAN_WRITE call, read by MX_PA_PLAN_READ
    int seg_slots;    // U: partial slots per segment window (the merge's batch)
};

// Slots per segment window, from the launch's workers and segments: 32 where segments are cut into
// more than about 10 pieces on average, else 16 (the merge then loads a window in one batch).
constexpr int seg_slots_for(int64_t workers, int64_t segs) { return workers > 10 * segs ? 32 : 16; }
constexpr int kPlanStride = 65;  // tile plan entries per worker: 64 tiles and a header {k of the first piece}

constexpr int kWaves = 4;               // waves per workgroup of the split launch (at most)
constexpr int kSmallWorkers = 1024;     // up to this many workers the split launch uses 2-wave workgroups
constexpr int kTile = 16;               // tokens per MFMA tile
constexpr int kMaxRangeTiles = 64;      // a worker's range fits one vector of block ids (block size >= 16)
// Tiles whose block ids fit one vector: block sizes 4 and 8 put 4 or 2 blocks in a tile.
constexpr int max_range_tiles(int block_size) {
    return block_size >= kTile ? kMaxRangeTiles : kMaxRangeTiles * block_size / kTile;
}
constexpr int kDefaultWorkers = 2048;   // 256 CUs x 8 waves on MI355X
constexpr int kMinDefaultTiles = 4;     // default ranges are at least this long when T allows
// Default workers per segment on average, but never fewer than one worker per CU. Measured on
// the Qwen2-0.5B shape (B 16, 2 kv-heads, contexts U[512, 2048]) with the 4-dims-per-thread
// merge: a cap of 8 pieces 14.4 us per call, 16 pieces 13.8 us, 32 pieces 15.3 us; re-measured
// with the unrolled short pieces (before the tile plan and the merge windows): 8 pieces 13.3 us,
// 12 13.05 us, 16 12.85 us, 24 15.2 us. At the Llama-3-8B bench shape (2048 workers) and for the
// 128-row batch (the range floor) the cap is not reached.
constexpr int kPiecesPerSegment = 16;
constexpr int kMinWorkers = 256;
constexpr int kMaxChunkTokens = kMaxRangeTiles * kTile;
constexpr float kLazyLog2 = 8.0f;       // rescale only when the running max rises by more than 2^8

__device__ __forceinline__ half8v load_half8(const _Float16* p) {
    return __builtin_bit_cast(half8v, *reinterpret_cast<const uint4*>(p));
}

// K/V loads. When every block id occurs in one row only, K and V are read once per call
// and STREAM = true issues non-temporal loads (the streaming cache policy), which keep
// them from displacing other lines: 62.0 -> 58.6-60.3 us per call at the batch-32 bench
// shape. When rows alias blocks (a shared prefix, MX_PA_SHARED_BLOCKS) the rows of a
// group read the same blocks at about the same time and STREAM = false keeps those
// re-reads in L2 / MALL: 402 -> 325 us per layer on the 128-row shared-prefix batch.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
template <bool STREAM>
__device__ __forceinline__ half8v load_kv8(const _Float16* p) {
    if constexpr (STREAM)
        return __builtin_bit_cast(half8v, __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p)));
    else
        return load_half8(p);
}
template <bool STREAM>
__device__ __forceinline__ half4v load_kv4(const _Float16* p) {
    if constexpr (STREAM)
        return __builtin_bit_cast(half4v, __builtin_nontemporal_load(reinterpret_cast<const u32x2v*>(p)));
    else
        return __builtin_bit_cast(half4v, *reinterpret_cast<const u32x2v*>(p));
}

// Element type of q, K, V and the output: fp16 (BF16 = false) or bf16 (MX_PA_BF16). Registers
// and memory hold the 16-bit patterns in half vectors either way; only the MFMA forms and the
// fp32 conversions differ. Probabilities enter P.V rounded to the element type, as the
// reference's SDPA path casts its softmax to the query dtype (paged_attention_triton.py:816).
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef short s16x4v __attribute__((ext_vector_type(4)));
template <bool BF16>
struct Elt;
template <>
struct Elt<false> {
    static __device__ __forceinline__ float4v mma32(half8v a, half8v b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float4v mma16(half4v a, half4v b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ _Float16 round(float x) { return (_Float16)x; }
    static __device__ __forceinline__ float widen(_Float16 x) { return (float)x; }
};
template <>
struct Elt<true> {
    static __device__ __forceinline__ float4v mma32(half8v a, half8v b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b),
                                                       c, 0, 0, 0);
    }
    static __device__ __forceinline__ float4v mma16(half4v a, half4v b, float4v c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4v, a), __builtin_bit_cast(s16x4v, b),
                                                         c, 0, 0, 0);
    }
    static __device__ __forceinline__ _Float16 round(float x) { return __builtin_bit_cast(_Float16, (__bf16)x); }
    static __device__ __forceinline__ float widen(_Float16 x) { return (float)__builtin_bit_cast(__bf16, x); }
};

// Tiles of row b (bounded by the table width) and its effective length.
template <int BS>
__device__ __forceinline__ int row_tiles(const Params& p, int b, int& s_eff) {
    const int S = p.seq_lens[b];
    int nblk = S > 0 ? (S + BS - 1) / BS : 0;
    if (nblk > p.max_blocks) nblk = p.max_blocks;
    s_eff = S < nblk * BS ? S : nblk * BS;
    return (s_eff + kTile - 1) / kTile;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

// Total tiles of all segments: Hkv * sum_b tiles(b).
template <int BS>
__device__ __forceinline__ int64_t total_tiles(const Params& p, int lane) {
    int64_t sum = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        int s_eff, n = 0;
        if (b0 + lane < p.B) n = row_tiles<BS>(p, b0 + lane, s_eff);
        sum += wave_sum_i(n);
    }
    return sum * p.Hkv;
}

struct Seg {
    int b, ntiles;
    int64_t row_start;  // global index of tile 0 of (b, kv-head 0)
};

// The row whose tiles contain global tile index x (x < total).
template <int BS>
__device__ __forceinline__ Seg locate(const Params& p, int64_t x, int lane) {
    int64_t base = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        int s_eff, n = 0;
        const bool valid = b0 + lane < p.B;
        if (valid) n = row_tiles<BS>(p, b0 + lane, s_eff);
        const int incl = wave_incl_scan(n, lane);
        const int64_t chunk_total = (int64_t)__builtin_amdgcn_readlane(incl, 63) * p.Hkv;
        if (x < base + chunk_total) {
            const int excl = incl - n;
            const bool le = valid && base + (int64_t)excl * p.Hkv <= x;
            const int bl = __builtin_popcountll(__builtin_amdgcn_ballot_w64(le)) - 1;
            return Seg{b0 + bl, __builtin_amdgcn_readlane(n, bl),
                       base + (int64_t)__builtin_amdgcn_readlane(excl, bl) * p.Hkv};
        }
        base += chunk_total;
    }
    return Seg{0, 0, 0};  // unreachable for x < total
}

__device__ __forceinline__ int64_t range_lo(int64_t w, int64_t T, int W) { return w * T / W; }

// V fragment of one token held by a lane: D/16 consecutive dims.
template <int D>
struct VFragT;
template <>
struct VFragT<128> {
    using type = half8v;
    template <bool STREAM>
    static __device__ __forceinline__ type load(const _Float16* p) { return load_kv8<STREAM>(p); }
};
template <>
struct VFragT<64> {
    using type = half4v;
    template <bool STREAM>
    static __device__ __forceinline__ type load(const _Float16* p) { return load_kv4<STREAM>(p); }
};

template <int KK, typename VF>
struct TileRegs {
    half8v k[KK];
    VF v[4];  // tokens 4*(lane/16) + j
};

// Tiles of K/V loads in flight per wave. Two keep the HBM queues full at the
// default worker count (a deeper pipeline measured slower on MI355X: more
// outstanding random 4 KiB runs per channel) and leave room for four waves
// per SIMD.
#ifndef MX_PA_DEPTH
#define MX_PA_DEPTH 2
#endif
constexpr int kDepth = MX_PA_DEPTH;

// At least 3 waves per SIMD: the compiler then keeps the kernel in 164 VGPRs without
// AGPRs (left free it used 166 + 36 and fit only 2). One round of 2048 workers stays the
// default; with the extra room per SIMD it measured 61.3 -> 60.1 us per call at the
// bench shape, while 3072 workers measured slower (62.1 us).
#ifndef MX_PA_MIN_WAVES
#define MX_PA_MIN_WAVES 3
#endif

// One piece: tiles [t0, t0 + nj) of segment (row b, kv-head kvh) with the row's effective length
// s_eff. Leaves the online-softmax state of query head r = lane % 16 of the kv-head's group in
// (m_run, l_run, acc): m_run on the exp2 scale, the same in all 4 lane groups; l_run this lane's
// partial denominator (sum over the 4 lane groups with xor_sum_16_32); acc[e][i] the
// unnormalised output of head r at dim (4g + i) * DPL + e, g = lane / 16. PROBE: the loads
// alone (see decode_split_kernel).
//
// PLANNED: the piece's block ids come from the plan (pb_in: lane j holds tile t0 + j's, -1 for an id
// outside the pool) instead of the block table. plan_dst (block size >= 16, not PLANNED): lanes
// j < nj also record their tile there as {block id, b << 16 | kvh, t0 + j, s_eff}.
template <int D, int BS, int G, bool STREAM, bool BF16, bool PROBE = false, bool PLANNED = false, int P = kDepth>
__device__ __forceinline__ void run_piece(const Params& p, int b, int kvh, int t0, int nj, int s_eff, int lane,
                                          float& m_run, float& l_run, float4v (&acc)[D / 16], int pb_in = 0,
                                          int4* plan_dst = nullptr) {
    constexpr int KK = D / 32;       // score MFMA k-steps over the head dim
    constexpr int DPL = D / 16;      // dims per lane in P.V: one MFMA per dim offset
    constexpr int TPB = BS >= kTile ? BS / kTile : 1;  // tiles per KV block (block sizes 16, 32)
    constexpr int BPT = BS >= kTile ? 1 : kTile / BS;  // KV blocks per tile (block sizes 4, 8)
    using VF = typename VFragT<D>::type;
    using Regs = TileRegs<KK, VF>;
    const float kNegInf = -__builtin_huge_valf();
    const int g = lane >> 4, r = lane & 15;
    const int h0 = kvh * G;
    // K: token r, dims 8g + 32kk; V: tokens 4g + j, dims DPL*r + e. With BPT > 1 a tile spans
    // BPT blocks: lane's K token lies in block slot kslot of the tile and its V tokens (and the
    // 4 scores it holds) in slot vslot, at the given offsets inside those blocks.
    const int koff = (BPT == 1 ? r : r % BS) * D + 8 * g;
    const int voff = (BPT == 1 ? 4 * g : (4 * g) % BS) * D + DPL * r;
    const int kslot = r / BS, vslot = (4 * g) / BS;

    // Block ids of the piece: lane j holds the id of tile t0 + j (BPT == 1) or of block
    // slot j of the piece's tiles (BPT > 1, only the row's blocks below s_eff are read);
    // an id outside the pool becomes -1 (its tokens skipped, error recorded).
    int my_pb = 0;
    if constexpr (PLANNED) {
        static_assert(BPT == 1, "the tile plan covers block sizes >= 16");
        my_pb = pb_in;
    } else {
        const int32_t* bt_row = p.bt + (int64_t)b * p.bt_sb;
        bool fetch;
        int bslot;
        if constexpr (BPT == 1) {
            fetch = lane < nj;
            bslot = (t0 + lane) / TPB;
        } else {
            bslot = t0 * BPT + lane;
            fetch = lane < nj * BPT && bslot < (s_eff + BS - 1) / BS;
        }
        if (fetch) {
            my_pb = bt_row[bslot];
            if ((unsigned)my_pb >= (unsigned)p.num_pool_blocks) {  // never read outside the pool
                atomicOr(p.err, 1);
                my_pb = -1;
            }
        }
        if constexpr (BPT == 1) {
            if (plan_dst && lane < nj) plan_dst[lane] = int4{my_pb, (int)((unsigned)b << 16 | (unsigned)kvh), t0 + lane, s_eff};
        }
    }

    // B operand: query head r (zero past G), dims 32*kk + 8*g + [0, 8).
    half8v qf[KK];
    if (r < G && !PROBE) {
        const _Float16* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(h0 + r) * p.q_sh + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qf[kk] = load_half8(qp + 32 * kk);
    } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qf[kk] = (_Float16)0.0f;
    }

    m_run = kNegInf;
    l_run = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    const _Float16* kbase = p.k + (int64_t)(kvh / p.vg) * p.kv_shead;
    const _Float16* vbase = p.v + (int64_t)(kvh / p.vg) * p.kv_shead;

    // Loads are unconditional: past the piece's last tile the index is clamped
    // (an L2 hit) and a skipped block reads block 0; only the compute below is
    // predicated, by wave-uniform flags, so waits count exact stages.
    auto load_tile = [&](int j, Regs& tr) {
        const int jc = j < nj ? j : nj - 1;
        const _Float16* kt;
        const _Float16* vt;
        if constexpr (BPT == 1) {
            const int pb = __builtin_amdgcn_readlane(my_pb, jc);
            const int t = t0 + jc;
            const int64_t base = (int64_t)(pb < 0 ? 0 : pb) * p.kv_sblk + (t % TPB) * kTile * D;
            kt = kbase + base;
            vt = vbase + base;
        } else {
            const int pk = __shfl(my_pb, jc * BPT + kslot);
            const int pv = __shfl(my_pb, jc * BPT + vslot);
            kt = kbase + (int64_t)(pk < 0 ? 0 : pk) * p.kv_sblk;
            vt = vbase + (int64_t)(pv < 0 ? 0 : pv) * p.kv_sblk;
        }
#pragma unroll
        // A K load reads 64 bytes of each of 16 token rows, half of each 128-byte line, and the
        // next load (kk + 1) reads the other halves. The first half goes out with the default
        // policy, so the line stays in L2 for its second reader; only that last read streams.
        // All-streaming K loads re-fetched about 9 MB of lines per call at the batch-32 bench
        // shape (split kernel 310.9 -> 301.8 MB fetched).
        for (int kk = 0; kk < KK; ++kk)
            tr.k[kk] = (kk & 1) == 0 ? load_half8(kt + koff + 32 * kk) : load_kv8<STREAM>(kt + koff + 32 * kk);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) tr.v[jj] = VFragT<D>::template load<STREAM>(vt + voff + jj * D);
    };

    auto compute_tile = [&](int j, const Regs& tr) {
        const int t = t0 + j;
        float4v s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) s = Elt<BF16>::mma32(tr.k[kk], qf[kk], s);
        // s[i] = score of token t*16 + 4g + i for head r.
        const int tok0 = t * kTile + 4 * g;
        // BPT > 1: this lane's 4 tokens lie in one block (slot vslot); a skipped block masks them.
        const bool skipped = BPT > 1 && __shfl(my_pb, j * BPT + vslot) < 0;
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = (tok0 + i < s_eff && !skipped) ? s[i] * p.scale_log2e : kNegInf;
        const float mx = xor_max_16_32(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
        // Lazy rescale: the reference point m_run moves only when a score exceeds it
        // by more than kLazyLog2, so p = exp2(s - m_run) <= 2^kLazyLog2 (exact range
        // for fp16, same relative rounding) and acc / l is unchanged. Rescaling all
        // accumulators at every new maximum cost ~100 instructions on most early tiles.
        const bool grow = mx > m_run + kLazyLog2;  // always true on the first tile
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = grow ? mx : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
            l_run *= alpha;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
            m_run = m_new;
        }
        half4v pv;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pv[i] = Elt<BF16>::round(__builtin_amdgcn_exp2f(sc[i] - m_run));
            // BPT > 1: every block of a tile may be outside the pool while m_run is still
            // -inf; exp2(-inf - -inf) is NaN, so masked scores give p = 0 explicitly.
            if constexpr (BPT > 1) pv[i] = sc[i] == kNegInf ? (_Float16)0.0f : pv[i];
            psum += Elt<BF16>::widen(pv[i]);
        }
        l_run += psum;
        // V rows past the sequence end are zeroed: p is 0 there, but stale pool
        // memory may hold Inf/NaN, and 0 * NaN would poison the sum.
        VF v[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) v[jj] = tr.v[jj];
        if (t * kTile + kTile > s_eff || skipped) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                if (tok0 + jj >= s_eff || skipped) v[jj] = VF{};
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const half4v a = {v[0][e], v[1][e], v[2][e], v[3][e]};
            acc[e] = Elt<BF16>::mma16(a, pv, acc[e]);
        }
    };

    if constexpr (PROBE) {
        Regs st[P];
        uint32_t sum = 0;
#pragma unroll
        for (int s = 0; s < P; ++s) load_tile(s, st[s]);
        for (int j0 = 0; j0 < nj; j0 += P) {
#pragma unroll
            for (int s = 0; s < P; ++s) {
                if (j0 + s < nj) {
                    const Regs& tr = st[s];
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) {
                        const uint4 w = __builtin_bit_cast(uint4, tr.k[kk]);
                        sum ^= w.x ^ w.y ^ w.z ^ w.w;
                    }
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const auto w = __builtin_bit_cast(typename std::conditional<D == 128, uint4, uint2>::type,
                                                          tr.v[jj]);
                        sum ^= w.x ^ w.y;
                    }
                }
                load_tile(j0 + s + P, st[s]);
            }
        }
        if (sum == 0x9e3779b9u) p.err[1] = (int)sum;  // keeps the loads; practically never taken
        return;
    }
    // Short pieces at D = 64 (the Qwen2-0.5B shape: ranges of about 5 tiles): every tile of the
    // piece in flight at once, then the unrolled compute, instead of P-deep rounds (one K/V round
    // trip instead of about three). 8 stages of 16 VGPRs fit beside the rest at 2 waves per SIMD,
    // enough for the default 2048 workers; at D = 128 they would not.
    constexpr int kUnrolled = (D == 64 && BPT == 1) ? 8 : 0;
    if constexpr (kUnrolled > 0) {
        if (nj <= kUnrolled) {
            Regs su[kUnrolled];
#pragma unroll
            for (int j = 0; j < kUnrolled; ++j)
                if (j < nj) load_tile(j, su[j]);
#pragma unroll
            for (int j = 0; j < kUnrolled; ++j)
                if (j < nj && __builtin_amdgcn_readlane(my_pb, j) >= 0) compute_tile(j, su[j]);
            return;
        }
    }
    {
        Regs st[P];
#pragma unroll
        for (int s = 0; s < P; ++s) load_tile(s, st[s]);
        for (int j0 = 0; j0 < nj; j0 += P) {
#pragma unroll
            for (int s = 0; s < P; ++s) {
                const int j = j0 + s;
                if (j < nj && (BPT > 1 || __builtin_amdgcn_readlane(my_pb, j) >= 0)) compute_tile(j, st[s]);
                load_tile(j + P, st[s]);
            }
        }
    }

}

// PROBE = true: the calibration instance of mx_kv_gather_probe. The same partition and the same
// K/V loads, with the math replaced by an xor of the loaded words (nothing is written unless
// that checksum hits a magic value), so its duration is the gather alone.
// PLAN: 0 a plain call, 1 a plain call that also records the tile plan (MX_PA_PLAN_WRITE), 2 a call
// that starts from the plan (MX_PA_PLAN_READ). The record's stores are in their own instance: in the
// plain one they pushed the D = 128 instances past their register budget (4-6 VGPRs of spills).
template <int D, int BS, int G, bool STREAM, bool BF16, bool PROBE = false, int PLAN = 0>
// The instance that records the tile plan (PLAN = 1, layer 0 of a decode step) and the block-size 4
// and 8 instances need more than the 168 VGPRs of 3 waves per SIMD (they spilled 12-28 bytes per
// lane there); at 2 waves per SIMD (256 VGPRs) they hold 171 without scratch and still keep the
// default 2048 workers resident in one round. The recording call at the bench shape: 60.7-61.6
// -> 56.8-56.9 us on MI355X (three interleaved pairs).
__global__ __launch_bounds__(kWaves * 64, ((D == 64 && !PROBE) || PLAN == 1 || BS < kTile) ? 2 : MX_PA_MIN_WAVES) void decode_split_kernel(Params p) {
    constexpr bool PLANNED = PLAN == 2;
    constexpr int DPL = D / 16;      // dims per lane in P.V: one MFMA per dim offset
    constexpr int BPT = BS >= kTile ? 1 : kTile / BS;  // KV blocks per tile (block sizes 4, 8)
    constexpr int kMaxRange = kMaxRangeTiles / BPT;    // tiles whose block ids fit one vector
    using VF = typename VFragT<D>::type;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int worker = blockIdx.x * p.wg_waves + wave;
    const int g = lane >> 4, r = lane & 15;

    // A finished piece: tiles [t0, t1) of segment (b, kvh), whose row has nt tiles, the segment's
    // k-th piece. A whole segment writes the output; a cut one its partial at slot seg*U + k of the
    // segment's window, or at the worker's overflow slot for k >= U.
    auto finish = [&](int b, int kvh, int t0, int t1, int nt, int64_t k, float m_run, float l_run,
                      const float4v (&acc)[DPL]) {
        const int h0 = kvh * G;
        // Denominator of head r over the 4 lane groups; acc already sums all 16 tokens of a tile.
        l_run = xor_sum_16_32(l_run);
        const bool whole = t0 == 0 && t1 == nt;
        const int64_t seg = (int64_t)b * p.Hkv + kvh;
        const int64_t slot = k < p.seg_slots ? seg * p.seg_slots + k : (int64_t)p.B * p.Hkv * p.seg_slots + worker;
        if (lane == 0) {
            if (t0 == 0) p.seg_w[2 * seg] = worker;
            if (t1 == nt) p.seg_w[2 * seg + 1] = worker;
        }
        if (r < G) {
            if (whole) {
                _Float16* orow = p.out + (int64_t)b * p.o_sb + (int64_t)(h0 + r) * p.o_sh;
                const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;  // 0: every block of the row was skipped
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    VF o;
#pragma unroll
                    for (int e = 0; e < DPL; ++e) o[e] = Elt<BF16>::round(acc[e][i] * inv);
                    *reinterpret_cast<VF*>(orow + (4 * g + i) * DPL) = o;
                }
            } else {
                // The piece's own normalised output, rounded to the element type: half the
                // bytes of the fp32 accumulator, and the merge re-weights it by l.
                _Float16* arow = p.part_out + (slot * G + r) * D;
                const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    VF o;
#pragma unroll
                    for (int e = 0; e < DPL; ++e) o[e] = Elt<BF16>::round(acc[e][i] * inv);
                    *reinterpret_cast<VF*>(arow + (4 * g + i) * DPL) = o;
                }
                if (g == 0) {
                    p.part_ml[(slot * G + r) * 2 + 0] = m_run;
                    p.part_ml[(slot * G + r) * 2 + 1] = l_run;
                }
            }
        }
    };

    if constexpr (PLANNED) {
        // The worker's tiles as a MX_PA_PLAN_WRITE call with the same lengths and tables recorded
        // them: lane j holds tile j of the range as {block id, b << 16 | kvh, t, s_eff} (-1 in the
        // second word past the range). One load replaces the lengths -> range -> block ids chain.
        // Entries are checked before use, so a plan that does not match the call reads nothing
        // outside the pool, q or the workspace; such pieces (also those whose row length changed
        // since, checked after their loads) write nothing and set error bit 8.
        const int4 e = p.plan[(int64_t)worker * kPlanStride + lane];
        const int k_first = p.plan[(int64_t)worker * kPlanStride + 64].x;
        const bool live = e.y != -1;
        const int prev_y = __shfl_up(e.y, 1), prev_t = __shfl_up(e.z, 1);
        const bool start = live && (lane == 0 || e.y != prev_y || e.z != prev_t + 1);
        uint64_t starts = __builtin_amdgcn_ballot_w64(start);
        const int count = __builtin_popcountll(__builtin_amdgcn_ballot_w64(live));
        while (starts) {
            const int j0 = (int)__builtin_ctzll(starts);
            starts &= starts - 1;
            const int j1 = starts ? (int)__builtin_ctzll(starts) : count;
            const unsigned bk = (unsigned)__builtin_amdgcn_readlane(e.y, j0);
            const int b = (int)(bk >> 16), kvh = (int)(bk & 0xffffu);
            const int t0 = __builtin_amdgcn_readlane(e.z, j0), s_eff = __builtin_amdgcn_readlane(e.w, j0);
            const int nj = j1 - j0;
            const int nt = (s_eff + kTile - 1) / kTile;
            // Only a worker's first piece can start inside its segment (k = k_first); the others
            // start their segments (k = 0).
            const int k = t0 == 0 ? 0 : k_first;
            if (b >= p.B || kvh >= p.Hkv || t0 < 0 || nj <= 0 || s_eff < 0 || s_eff > p.max_blocks * BS ||
                t0 + nj > nt || (t0 > 0 && (j0 != 0 || k < 1 || k > worker))) {
                if (lane == 0) atomicOr(p.err, 8);
                break;
            }
            int pb = __shfl(e.x, j0 + lane);
            if (lane >= nj || (unsigned)pb >= (unsigned)p.num_pool_blocks) pb = -1;
            float m_run, l_run;
            float4v acc[DPL];
            run_piece<D, BS, G, STREAM, BF16, false, true>(p, b, kvh, t0, nj, s_eff, lane, m_run, l_run, acc, pb);
            int s_now;
            row_tiles<BS>(p, b, s_now);
            if (s_now != s_eff) {  // the row's length changed since the plan was recorded
                if (lane == 0) atomicOr(p.err, 8);
                continue;
            }
            finish(b, kvh, t0, t0 + nj, nt, k, m_run, l_run, acc);
        }
        return;
    }

    // Up to 64 rows: one read of seq_lens per wave, reused to locate every piece.
    const bool one_pass = p.B <= 64;
    int n_lane = 0, s_eff_lane = 0, incl_lane = 0;
    int64_t T;
    if (one_pass) {
        if (lane < p.B) n_lane = row_tiles<BS>(p, lane, s_eff_lane);
        incl_lane = wave_incl_scan(n_lane, lane);
        T = (int64_t)__builtin_amdgcn_readlane(incl_lane, 63) * p.Hkv;
    } else {
        T = total_tiles<BS>(p, lane);
    }
    const int W = T < p.workers ? (int)T : p.workers;  // every worker gets >= 1 tile
    // MX_PA_PLAN_WRITE (block size >= 16): record every tile of the range for later calls; lanes
    // past the range (all of them for an idle worker) mark the end.
    int4* const plan_w = (PLAN == 1 && !PROBE && BPT == 1) ? p.plan + (int64_t)worker * kPlanStride : nullptr;
    if (worker >= W) {
        if (plan_w) plan_w[lane] = int4{0, -1, 0, 0};
        return;
    }
    const int64_t hi = range_lo(worker + 1, T, W);
    int64_t x = range_lo(worker, T, W);
    const int64_t x_first = x;
    if (plan_w && lane >= hi - x_first) plan_w[lane] = int4{0, -1, 0, 0};

    // The segment holding global tile xx, from the lengths read above (or read again past 64 rows).
    auto seg_at = [&](int64_t xx) {
        if (one_pass) {
            const int excl = incl_lane - n_lane;
            const bool le = lane < p.B && (int64_t)excl * p.Hkv <= xx;
            const int bl = __builtin_popcountll(__builtin_amdgcn_ballot_w64(le)) - 1;
            return Seg{bl, __builtin_amdgcn_readlane(n_lane, bl), (int64_t)__builtin_amdgcn_readlane(excl, bl) * p.Hkv};
        }
        return locate<BS>(p, xx, lane);
    };
    // Index of the worker's first piece within its segment: 0 when the range starts a segment;
    // otherwise this worker minus the one holding the segment's first tile xs,
    // floor(((xs + 1) W - 1) / T), the w with range_lo(w) <= xs < range_lo(w + 1). Every later
    // piece starts its segment (index 0). Computed here, so that T and W are not held through
    // the pieces (that pushed the D = 128 instances into spills).
    int k_first = 0;
    if (!PROBE) {
        const Seg s0 = seg_at(x_first);
        if (s0.ntiles > 0) {
            const int64_t t00 = (x_first - s0.row_start) % s0.ntiles;
            if (t00 > 0) k_first = (int)(worker - ((x_first - t00 + 1) * W - 1) / T);
        }
        if (plan_w && lane == 0) plan_w[64] = int4{k_first, 0, 0, 0};
    }

    while (x < hi) {
        const Seg sg = seg_at(x);
        const int b = sg.b, nt = sg.ntiles;
        if (nt <= 0) {  // cannot happen for x < T; stop rather than divide by zero
            atomicOr(p.err, 4);
            break;
        }
        const int kvh = (int)((x - sg.row_start) / nt);
        const int t0 = (int)((x - sg.row_start) % nt);
        const int t1 = (int64_t)(nt - t0) < hi - x ? nt : (int)(t0 + (hi - x));
        const int nj = t1 - t0;  // <= kMaxRange because W >= ceil(T_max / kMaxRange)
        if (nj > kMaxRange) {
            atomicOr(p.err, 4);
            break;
        }
        int4* const plan_dst = plan_w ? plan_w + (x - x_first) : nullptr;
        x += nj;
        int s_eff;
        if (one_pass) s_eff = __builtin_amdgcn_readlane(s_eff_lane, b);
        else row_tiles<BS>(p, b, s_eff);
        float m_run, l_run;
        float4v acc[DPL];
        run_piece<D, BS, G, STREAM, BF16, PROBE>(p, b, kvh, t0, nj, s_eff, lane, m_run, l_run, acc, 0, plan_dst);
        if constexpr (PROBE) continue;
        finish(b, kvh, t0, t1, nt, t0 > 0 ? k_first : 0, m_run, l_run, acc);
    }
}

// Log-sum-exp merge of the partials of one (kv-head, sequence); zeros for an empty row.
// Workers seg_w[s] .. seg_w[s + 1] cut segment s; piece k's partial is at slot s*U + k of the
// segment's window, or at overflow slot B*Hkv*U + seg_w[s] + k for k >= U.
// Thread t owns 4 consecutive dims of one head (16-byte partial loads; m and l are shared
// by the head's threads).
template <int D, int G>
constexpr int merge_threads() {
    return ((G * D / 4 + 63) / 64) * 64;
}

// One batch of the online log-sum-exp: the UB pieces' (m, l) and normalised outputs, of which the
// first cnt are real (the rest masked). Branch-free, so that loads issued before it are not
// sunk behind anything.
template <int UB, bool BF16>
__device__ __forceinline__ void merge_step(const float (&mv)[UB], const float (&lv)[UB], const half4v (&av)[UB],
                                           int cnt, float& mg, float& l, float4v& a) {
    const float kNegInf = -__builtin_huge_valf();
    float mc = kNegInf;
#pragma unroll
    for (int u = 0; u < UB; ++u) mc = u < cnt ? fmaxf(mc, mv[u]) : mc;
    const float mn = fmaxf(mg, mc);
    const bool any = mn != kNegInf;  // false while every tile so far was skipped
    const float r = any ? exp2f(mg - mn) : 1.0f;
    l *= r;
    a *= r;
    // Masked slots may hold anything (an earlier call's pieces, NaN): their terms are selected
    // away, never multiplied by 0.
#pragma unroll
    for (int u = 0; u < UB; ++u) {
        const bool v = u < cnt && any;
        const float wgt = exp2f(mv[u] - mn) * lv[u];
        l = v ? l + wgt : l;
        const float4v o = {Elt<BF16>::widen(av[u][0]), Elt<BF16>::widen(av[u][1]), Elt<BF16>::widen(av[u][2]),
                           Elt<BF16>::widen(av[u][3])};
        const float4v t = a + wgt * o;  // the piece's output, normalised by its own l
        a = v ? t : a;
    }
    mg = any ? mn : mg;
}

// U: slots per segment window and partials loaded per memory round trip (Params::seg_slots).
template <int D, int BS, int G, bool BF16, int U = 16>
__global__ __launch_bounds__(256) void decode_merge_kernel(Params p) {
    constexpr int Q = D / 4;  // 4-dim groups per head
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x;
    const bool active = tid < G * Q;
    const int h = active ? tid / Q : 0, d = active ? (tid % Q) * 4 : 0;
    const int64_t s = (int64_t)b * p.Hkv + kvh;
    // Every load of the common case goes out at once: the row's length, the segment's worker span
    // and the segment's whole window (slots that hold no piece of this call are loaded and masked).
    int s_eff;
    const int nt = row_tiles<BS>(p, b, s_eff);
    const int w0 = p.seg_w[2 * s], w1 = p.seg_w[2 * s + 1];
    float mv[U], lv[U];
    half4v av[U];  // 16-bit until used: half the registers of fp32
    {
        const float* mlp = p.part_ml + ((s * U) * G + h) * 2;
        const _Float16* accp = p.part_out + ((s * U) * G + h) * D + d;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            mv[u] = mlp[u * G * 2];
            lv[u] = mlp[u * G * 2 + 1];
            av[u] = *reinterpret_cast<const half4v*>(accp + u * G * D);
        }
    }
    // Keep the scheduler from interleaving the window's loads with the math below (it would
    // issue the later ones only after the first ones are consumed).
    __builtin_amdgcn_sched_barrier(0);
    // Pieces of this call: none for an empty row or a segment one worker held whole (that worker
    // wrote the output; nothing is stored here).
    const bool whole = nt > 0 && w0 == w1;
    const int np = (nt == 0 || whole || w1 < w0) ? 0 : w1 - w0 + 1;
    const float kNegInf = -__builtin_huge_valf();
    float mg = kNegInf, l = 0.0f;
    float4v a = {0.0f, 0.0f, 0.0f, 0.0f};
    merge_step<U, BF16>(mv, lv, av, np < U ? np : U, mg, l, a);
    // Segments of more than U pieces: the rest from the overflow slots of their workers.
    const int64_t ovf = (int64_t)p.B * p.Hkv * U;
    for (int i0 = U; i0 < np; i0 += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u < np ? i0 + u : np - 1;
            const int64_t slot = ovf + w0 + i;
            mv[u] = p.part_ml[(slot * G + h) * 2];
            lv[u] = p.part_ml[(slot * G + h) * 2 + 1];
            av[u] = *reinterpret_cast<const half4v*>(p.part_out + (slot * G + h) * D + d);
        }
        merge_step<U, BF16>(mv, lv, av, np - i0 < U ? np - i0 : U, mg, l, a);
    }
    if (active && !whole) {
        half4v o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = Elt<BF16>::round(l > 0.0f ? a[e] / l : 0.0f);
        _Float16* out = p.out + (int64_t)b * p.o_sb + (int64_t)(kvh * G + h) * p.o_sh + d;
        *reinterpret_cast<half4v*>(out) = o;
    }
}

// GQA groups above 8 (the kernels' largest G) are served as virtual kv-heads: pool head k
// becomes heads k * vg .. k * vg + vg - 1 of G / vg query heads each (query head order is
// unchanged), with vg the smallest divisor of G that brings the group to 8 or fewer. Each
// virtual head reads its pool head's K/V, so K/V bytes are read vg times (the reference's
// kernels read them G times, paged_attention_triton.py:179-181).
static inline int kv_virtual_groups(int Hq, int Hkv) {
    const int G = Hkv > 0 ? Hq / Hkv : 1;
    for (int vg = 1; vg <= G; ++vg)
        if (G % vg == 0 && G / vg <= 8) return vg;
    return G;
}

struct Layout {
    size_t err, segw, ml, acc, plan, total;  // plan == total: no tile plan in this layout
    int workers;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Number of workers. T_max (every row at the table width) bounds the real tile
// count, so W >= ceil(T_max / max_range_tiles) keeps each range within one vector
// of block ids. chunk_tokens > 0 asks for ranges of about that many tokens at T_max;
// 0 picks kDefaultWorkers (one round of resident waves on the chip), fewer
// when that would make ranges shorter than kMinDefaultTiles tiles or cut a
// segment into more than kPiecesPerSegment pieces on average (but at least
// kMinWorkers).
static int resolve_workers(int chunk_tokens, int B, int Hkv, int max_blocks, int block_size) {
    const int64_t row_tiles_max = ceil_div((int64_t)max_blocks * block_size, kTile);
    const int64_t t_max = (int64_t)B * Hkv * row_tiles_max;
    const int64_t floor_w = ceil_div(t_max, max_range_tiles(block_size));
    int64_t w;
    if (chunk_tokens > 0) {
        w = ceil_div(t_max, chunk_tokens / kTile);
    } else {
        w = ceil_div(t_max, kMinDefaultTiles);
        const int64_t per_seg = (int64_t)B * Hkv * kPiecesPerSegment;
        const int64_t cap = per_seg > kMinWorkers ? per_seg : kMinWorkers;
        if (w > cap) w = cap;
        if (w > kDefaultWorkers) w = kDefaultWorkers;
    }
    if (w < floor_w) w = floor_w;
    if (w < 1) w = 1;
    return (int)(w > (1 << 30) ? (1 << 30) : w);
}

// Hkv: kv-heads as the kernels see them (after kv_virtual_groups). with_plan: room for the tile
// plan of MX_PA_PLAN_WRITE / MX_PA_PLAN_READ (64 entries of 16 bytes per worker, block size >= 16).
static Layout layout(int B, int Hq, int Hkv, int D, int max_blocks, int block_size, int chunk_tokens,
                     bool with_plan) {
    Layout L{};
    L.workers = resolve_workers(chunk_tokens, B, Hkv, max_blocks, block_size);
    const int G = Hkv > 0 ? Hq / Hkv : 0;
    // Segment windows (U slots each, U for the uncapped worker count: a launch that caps its
    // workers never uses a larger U) and one overflow slot per worker.
    const size_t slots = (size_t)B * Hkv * seg_slots_for(L.workers, (int64_t)B * Hkv) + (size_t)L.workers;
    L.err = 0;
    L.segw = 256;
    L.ml = L.segw + align256((size_t)B * Hkv * 2 * sizeof(int));
    L.acc = L.ml + align256(slots * G * 2 * sizeof(float));
    L.plan = L.acc + align256(slots * G * D * sizeof(uint16_t));
    L.total = L.plan + (with_plan && block_size >= kTile ? align256((size_t)L.workers * kPlanStride * sizeof(int4)) : 0);
    return L;
}

// Waves of this kernel instance that fit on the current device at once
// (occupancy x CUs), cached per device; 0 if the runtime cannot say.
template <int D, int BS, int G, bool STREAM, bool BF16>
static int resident_waves() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cache[dev] == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_split_kernel<D, BS, G, STREAM, BF16>, kWaves * 64, 0) !=
                hipSuccess)
            return 0;
        cache[dev] = cus * per_cu * kWaves;
    }
    return cache[dev];
}

template <int D, int BS, int G, bool STREAM, bool BF16, int PLAN = 0>
static void launch(Params prm, int B, hipStream_t st, int64_t floor_workers) {
    // The worker count comes from the plain instance, so a MX_PA_PLAN_READ call has exactly the
    // workers whose plans the MX_PA_PLAN_WRITE call recorded.
    // More workers than resident waves would leave a second, partial round; use
    // one round unless ranges would then exceed max_range_tiles.
    const int cap = resident_waves<D, BS, G, STREAM, BF16>();
    if (cap > 0 && prm.workers > cap) prm.workers = (int)(floor_workers > cap ? floor_workers : cap);
    // Up to kSmallWorkers workers, 2-wave workgroups spread the waves over twice as many CUs (one
    // CU streams at most ~55 GB/s of this gather): Qwen2-0.5B shape, 512 workers, 13.8-14.2 ->
    // 13.4-13.5 us per call on MI355X. With 2048 workers, 4-wave workgroups measured 56.0 us against
    // 56.3 (2 waves) and 57.3 (1 wave).
    prm.wg_waves = prm.workers <= kSmallWorkers ? 2 : kWaves;
    prm.seg_slots = seg_slots_for(prm.workers, (int64_t)B * prm.Hkv);
    const int blocks = (int)ceil_div(prm.workers, prm.wg_waves);
    hipLaunchKernelGGL((decode_split_kernel<D, BS, G, STREAM, BF16, false, PLAN>), dim3(blocks),
                       dim3(prm.wg_waves * 64), 0, st, prm);
    const int64_t segs = (int64_t)B * prm.Hkv;
    if (seg_slots_for(prm.workers, segs) == 32)
        hipLaunchKernelGGL((decode_merge_kernel<D, BS, G, BF16, 32>), dim3(prm.Hkv, B), dim3(merge_threads<D, G>()), 0,
                           st, prm);
    else
        hipLaunchKernelGGL((decode_merge_kernel<D, BS, G, BF16, 16>), dim3(prm.Hkv, B), dim3(merge_threads<D, G>()), 0,
                           st, prm);
}

template <int D, int BS, bool STREAM, bool BF16, int PLAN>
static bool dispatch_plan_g(int G, const Params& prm, int B, hipStream_t st, int64_t fw) {
    switch (G) {
        case 1: launch<D, BS, 1, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 2: launch<D, BS, 2, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 3: launch<D, BS, 3, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 4: launch<D, BS, 4, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 5: launch<D, BS, 5, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 6: launch<D, BS, 6, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 7: launch<D, BS, 7, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        case 8: launch<D, BS, 8, STREAM, BF16, PLAN>(prm, B, st, fw); return true;
        default: return false;
    }
}

// plan: 0 plain, 1 record the tile plan, 2 start from it (block sizes >= 16, streaming loads only).
template <int D, int BS, bool STREAM, bool BF16>
static bool dispatch_g(int G, int plan, const Params& prm, int B, hipStream_t st, int64_t fw) {
    if (plan != 0) {
        if constexpr (BS >= kTile && STREAM) {
            return plan == 1 ? dispatch_plan_g<D, BS, STREAM, BF16, 1>(G, prm, B, st, fw)
                             : dispatch_plan_g<D, BS, STREAM, BF16, 2>(G, prm, B, st, fw);
        }
        return false;
    }
    return dispatch_plan_g<D, BS, STREAM, BF16, 0>(G, prm, B, st, fw);
}

template <bool STREAM, bool BF16>
static bool dispatch_d_bs(int D, int BS, int G, int plan, const Params& prm, int B, hipStream_t st, int64_t fw) {
    switch (D * 100 + BS) {
        case 12804: return dispatch_g<128, 4, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 12808: return dispatch_g<128, 8, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 12816: return dispatch_g<128, 16, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 12832: return dispatch_g<128, 32, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 6404: return dispatch_g<64, 4, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 6408: return dispatch_g<64, 8, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 6416: return dispatch_g<64, 16, STREAM, BF16>(G, plan, prm, B, st, fw);
        case 6432: return dispatch_g<64, 32, STREAM, BF16>(G, plan, prm, B, st, fw);
        default: return false;
    }
}

// Whole-block gather (mx_kv_gather_probe mode 1): the tiles of every row, flattened row-major,
// cut into equal ranges, one per workgroup of Hkv waves; wave h reads the K and V runs of head h
// of each tile's block, so a workgroup requests a block's Hkv runs (contiguous in the pool)
// together. Two tiles in flight per wave, streaming loads, xor checksum as in PROBE.
template <int D>
__global__ __launch_bounds__(1024) void kv_block_probe_kernel(Params p) {
    constexpr int RUN16 = D * kTile * 2 / 16;  // 16-byte chunks in one (tile, head) run: 256 at D 128
    constexpr int U = RUN16 / 64;              // chunks per lane per run
    const int lane = threadIdx.x & 63, h = threadIdx.x >> 6;
    int64_t T = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {  // tiles of all rows (kv-head 0 only)
        int s_eff, n = 0;
        if (b0 + lane < p.B) n = row_tiles<kTile>(p, b0 + lane, s_eff);
        T += wave_sum_i(n);
    }
    const int W = T < (int64_t)gridDim.x ? (int)T : (int)gridDim.x;
    if ((int)blockIdx.x >= W) return;
    int64_t x = range_lo(blockIdx.x, T, W);
    const int64_t hi = range_lo(blockIdx.x + 1, T, W);
    uint32_t sum = 0;
    while (x < hi) {
        // Row of tile x: locate with Hkv = 1 (tiles counted once per row).
        Params q1 = p;
        q1.Hkv = 1;
        const Seg sg = locate<kTile>(q1, x, lane);
        const int t0 = (int)(x - sg.row_start);
        const int nj = (int)((int64_t)(sg.ntiles - t0) < hi - x ? sg.ntiles - t0 : hi - x);
        const int32_t* bt_row = p.bt + (int64_t)sg.b * p.bt_sb;
        uint4 r[2][2 * U];
        auto load = [&](int j, uint4* d) {
            const int jc = j < nj ? j : nj - 1;
            const int t = t0 + jc;
            int pb = bt_row[t];  // block size 16: tile t is block t of the row
            pb = (unsigned)pb < (unsigned)p.num_pool_blocks ? pb : 0;
            const uint4* kp = reinterpret_cast<const uint4*>(p.k + (int64_t)pb * p.kv_sblk + (int64_t)h * p.kv_shead);
            const uint4* vp = reinterpret_cast<const uint4*>(p.v + (int64_t)pb * p.kv_sblk + (int64_t)h * p.kv_shead);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const u32x4v a = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(kp + u * 64 + lane));
                const u32x4v c = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(vp + u * 64 + lane));
                d[u] = uint4{a.x, a.y, a.z, a.w};
                d[U + u] = uint4{c.x, c.y, c.z, c.w};
            }
        };
        load(0, r[0]);
        load(1, r[1]);
        for (int j0 = 0; j0 < nj; j0 += 2) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                if (j0 + s < nj) {
#pragma unroll
                    for (int u = 0; u < 2 * U; ++u) sum ^= r[s][u].x ^ r[s][u].y ^ r[s][u].z ^ r[s][u].w;
                }
                load(j0 + s + 2, r[s]);
            }
        }
        x += nj;
    }
    if (sum == 0x9e3779b9u) p.err[1] = (int)sum;
}

}  // namespace pa
}  // namespace mx

using namespace mx;

extern "C" size_t mx_paged_attn_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                                int32_t block_size, int32_t chunk_tokens) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_blocks < 0 || block_size <= 0) return 0;
    return pa::layout(B, Hq, Hkv * pa::kv_virtual_groups(Hq, Hkv), D, max_blocks, block_size, chunk_tokens, true).total;
}

extern "C" size_t mx_paged_attn_error_offset(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_blocks,
                                             int32_t block_size, int32_t chunk_tokens) {
    if (Hkv <= 0) return 0;
    return pa::layout(B, Hq, Hkv * pa::kv_virtual_groups(Hq, Hkv), D, max_blocks, block_size, chunk_tokens, true).err;
}

namespace mx {
namespace pa {

// Argument checks shared by the two decode entry points; fills the launch parameters except
// the workspace pointers.
static int check_args(const char* what, const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                      const uint16_t* v, int64_t kv_sblk, int64_t kv_shead, const int32_t* block_tables, int64_t bt_sb,
                      int32_t max_blocks, const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                      int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out, int64_t o_sb,
                      int64_t o_sh, int32_t chunk_tokens, uint32_t flags, Params& prm) {
    if (!q || !k || !v || !block_tables || !seq_lens || !out) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
        return fail(MX_ERR_INVALID, "%s: Hq (%d) must be a positive multiple of Hkv (%d)", what, Hq, Hkv);
    if (D != 64 && D != 128) return fail(MX_ERR_UNSUPPORTED, "%s: head_dim %d unsupported", what, D);
    if (block_size != 4 && block_size != 8 && block_size != 16 && block_size != 32)
        return fail(MX_ERR_UNSUPPORTED, "%s: block_size %d unsupported (4, 8, 16 or 32)", what, block_size);
    if (max_blocks < 1 || num_pool_blocks < 1)
        return fail(MX_ERR_INVALID, "%s: max_blocks and num_pool_blocks must be >= 1", what);
    const int vg = kv_virtual_groups(Hq, Hkv);
    if (B > 65535 || (int64_t)Hkv * vg > 65535) return fail(MX_ERR_UNSUPPORTED, "%s: B or Hq too large", what);
    if (flags & ~(uint32_t)(MX_PA_SHARED_BLOCKS | MX_PA_BF16 | MX_PA_PLAN_WRITE | MX_PA_PLAN_READ))
        return fail(MX_ERR_INVALID, "%s: unknown flags 0x%x", what, flags);
    if ((flags & MX_PA_PLAN_WRITE) && (flags & MX_PA_PLAN_READ))
        return fail(MX_ERR_INVALID, "%s: MX_PA_PLAN_WRITE and MX_PA_PLAN_READ exclude each other", what);
    if ((flags & (MX_PA_PLAN_WRITE | MX_PA_PLAN_READ)) && (block_size < kTile || (flags & MX_PA_SHARED_BLOCKS)))
        return fail(MX_ERR_UNSUPPORTED, "%s: the tile plan needs block_size >= 16 and no MX_PA_SHARED_BLOCKS", what);
    if (chunk_tokens < 0 || chunk_tokens % kTile != 0 || chunk_tokens > kMaxChunkTokens)
        return fail(MX_ERR_INVALID, "%s: chunk_tokens must be 0 or a multiple of 16 <= %d", what, kMaxChunkTokens);
    if ((int64_t)B * Hkv * vg * ceil_div((int64_t)max_blocks * block_size, kTile) > ((int64_t)1 << 31))
        return fail(MX_ERR_UNSUPPORTED, "%s: more than 2^31 tiles", what);
    if (!aligned(q, 16) || q_sb % 8 || q_sh % 8 || !aligned(k, 16) || !aligned(v, 16) || kv_sblk % 8 ||
        kv_shead % 8 || !aligned(out, 16) || o_sb % 8 || o_sh % 8)
        return fail(MX_ERR_ALIGNMENT, "%s: q/K/V/out rows must be 16-byte aligned", what);
    prm = Params{};
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
    prm.B = B;
    prm.Hkv = Hkv * vg;  // kv-heads as the kernels see them
    prm.vg = vg;
    prm.num_pool_blocks = num_pool_blocks;
    prm.scale_log2e = scale * 1.4426950408889634f;
    prm.out = reinterpret_cast<_Float16*>(out);
    prm.o_sb = o_sb;
    prm.o_sh = o_sh;
    return MX_OK;
}

// Points the launch at a workspace laid out by `L` (err may redirect the error word) and launches.
static int launch_decode(const char* what, Params prm, const Layout& L, char* ws, int32_t* err, int32_t B, int32_t Hq,
                         int32_t Hkv, int32_t D, int32_t max_blocks, int32_t block_size, uint32_t flags, void* stream) {
    const int G = Hq / Hkv;
    prm.err = err ? err : reinterpret_cast<int*>(ws + L.err);
    prm.part_ml = reinterpret_cast<float*>(ws + L.ml);
    prm.part_out = reinterpret_cast<_Float16*>(ws + L.acc);
    prm.seg_w = reinterpret_cast<int*>(ws + L.segw);
    prm.plan = (flags & (MX_PA_PLAN_WRITE | MX_PA_PLAN_READ)) ? reinterpret_cast<int4*>(ws + L.plan) : nullptr;
    prm.workers = L.workers;
    hipStream_t st = as_stream(stream);
    // Fewest workers that keep every range within one vector of block ids.
    const int64_t fw = ceil_div((int64_t)B * Hkv * ceil_div((int64_t)max_blocks * block_size, kTile),
                                max_range_tiles(block_size));
    const bool shared = flags & MX_PA_SHARED_BLOCKS, bf16 = flags & MX_PA_BF16;
    const int plan = (flags & MX_PA_PLAN_READ) ? 2 : ((flags & MX_PA_PLAN_WRITE) ? 1 : 0);
    bool ok;
    if (bf16)
        ok = shared ? dispatch_d_bs<false, true>(D, block_size, G, plan, prm, B, st, fw)
                    : dispatch_d_bs<true, true>(D, block_size, G, plan, prm, B, st, fw);
    else
        ok = shared ? dispatch_d_bs<false, false>(D, block_size, G, plan, prm, B, st, fw)
                    : dispatch_d_bs<true, false>(D, block_size, G, plan, prm, B, st, fw);
    if (!ok) return fail(MX_ERR_UNSUPPORTED, "%s: unsupported configuration", what);
    return check_launch(what);
}

// Scratch of mx_paged_attn_decode_noalloc: a file-scope device array, one copy per GPU, held
// until the process ends. Host code never passes the array's name to a kernel (on the host it
// is a stand-in, not a device address): each device's address comes from hipGetSymbolAddress,
// taken once per device with that device current, and only that pointer is used.
static __device__ __align__(256) char scratch[MX_PA_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_of_current_device(char** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MX_ERR_LAUNCH, "mx_paged_attn_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(MX_ERR_UNSUPPORTED, "mx_paged_attn_decode_noalloc: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MX_ERR_LAUNCH, "mx_paged_attn_decode_noalloc: hipGetSymbolAddress(scratch): %s",
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = static_cast<char*>(g_scratch_ptr[dev]);
    return MX_OK;
}

}  // namespace pa
}  // namespace mx

extern "C" int mx_paged_attn_decode(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                                    const uint16_t* v, int64_t kv_sblk, int64_t kv_shead,
                                    const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                    const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                    int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out,
                                    int64_t o_sb, int64_t o_sh, void* workspace, size_t workspace_bytes,
                                    int32_t chunk_tokens, uint32_t flags, void* stream) {
    const char* what = "mx_paged_attn_decode";
    if (B < 0) return fail(MX_ERR_INVALID, "%s: B must be >= 0", what);
    if (B == 0) return MX_OK;
    pa::Params prm;
    int rc = pa::check_args(what, q, q_sb, q_sh, k, v, kv_sblk, kv_shead, block_tables, bt_sb, max_blocks, seq_lens, B,
                            Hq, Hkv, D, block_size, num_pool_blocks, scale, out, o_sb, o_sh, chunk_tokens, flags, prm);
    if (rc != MX_OK) return rc;
    const pa::Layout L = pa::layout(B, Hq, prm.Hkv, D, max_blocks, block_size, chunk_tokens, true);
    if (!workspace || workspace_bytes < L.total)
        return fail(MX_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", what, L.total, workspace_bytes);
    if (!aligned(workspace, 256)) return fail(MX_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", what);
    return pa::launch_decode(what, prm, L, static_cast<char*>(workspace), nullptr, B, Hq, prm.Hkv, D, max_blocks,
                             block_size, flags, stream);
}

extern "C" int mx_paged_attn_decode_noalloc(const uint16_t* q, int64_t q_sb, int64_t q_sh, const uint16_t* k,
                                            const uint16_t* v, int64_t kv_sblk, int64_t kv_shead,
                                            const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                            const int32_t* seq_lens, int32_t B, int32_t Hq, int32_t Hkv, int32_t D,
                                            int32_t block_size, int32_t num_pool_blocks, float scale, uint16_t* out,
                                            int64_t o_sb, int64_t o_sh, int32_t chunk_tokens, uint32_t flags,
                                            int32_t* err, void* stream) {
    const char* what = "mx_paged_attn_decode_noalloc";
    if (B < 0) return fail(MX_ERR_INVALID, "%s: B must be >= 0", what);
    if (B == 0) return MX_OK;
    pa::Params prm;
    int rc = pa::check_args(what, q, q_sb, q_sh, k, v, kv_sblk, kv_shead, block_tables, bt_sb, max_blocks, seq_lens, B,
                            Hq, Hkv, D, block_size, num_pool_blocks, scale, out, o_sb, o_sh, chunk_tokens, flags, prm);
    if (rc != MX_OK) return rc;
    if (err && !aligned(err, 4)) return fail(MX_ERR_ALIGNMENT, "%s: err must be 4-byte aligned", what);
    if (flags & (MX_PA_PLAN_WRITE | MX_PA_PLAN_READ))
        return fail(MX_ERR_INVALID, "%s: the tile plan lives in a caller's workspace (mx_paged_attn_decode)", what);
    const pa::Layout L = pa::layout(B, Hq, prm.Hkv, D, max_blocks, block_size, chunk_tokens, false);
    if (L.total > (size_t)MX_PA_NOALLOC_SCRATCH_BYTES)
        return fail(MX_ERR_WORKSPACE, "%s: this shape needs %zu bytes of scratch, more than the %zu the library holds "
                                      "per GPU; use mx_paged_attn_decode with a workspace",
                    what, L.total, (size_t)MX_PA_NOALLOC_SCRATCH_BYTES);
    char* ws = nullptr;
    rc = pa::scratch_of_current_device(&ws);
    if (rc != MX_OK) return rc;
    return pa::launch_decode(what, prm, L, ws, err, B, Hq, prm.Hkv, D, max_blocks, block_size, flags, stream);
}

extern "C" int mx_kv_gather_probe(const uint16_t* k, const uint16_t* v, int64_t kv_sblk, int64_t kv_shead,
                                  const int32_t* block_tables, int64_t bt_sb, int32_t max_blocks,
                                  const int32_t* seq_lens, int32_t B, int32_t Hkv, int32_t D, int32_t block_size,
                                  int32_t num_pool_blocks, int32_t mode, int32_t* sink, void* stream) {
    const char* what = "mx_kv_gather_probe";
    if (B < 0) return fail(MX_ERR_INVALID, "%s: B must be >= 0", what);
    if (B == 0) return MX_OK;
    if (!k || !v || !block_tables || !seq_lens || !sink) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (D != 64 && D != 128) return fail(MX_ERR_UNSUPPORTED, "%s: head_dim %d unsupported", what, D);
    if (block_size != 16 || Hkv < 1 || Hkv > 16 || max_blocks < 1 || num_pool_blocks < 1)
        return fail(MX_ERR_UNSUPPORTED, "%s: needs block_size 16, 1 <= Hkv <= 16", what);
    if (mode != 0 && mode != 1) return fail(MX_ERR_INVALID, "%s: mode must be 0 or 1", what);
    if (!aligned(k, 16) || !aligned(v, 16) || kv_sblk % 8 || kv_shead % 8 || !aligned(sink, 8))
        return fail(MX_ERR_ALIGNMENT, "%s: K/V runs must be 16-byte aligned", what);
    pa::Params prm{};
    prm.k = reinterpret_cast<const _Float16*>(k);
    prm.v = reinterpret_cast<const _Float16*>(v);
    prm.kv_sblk = kv_sblk;
    prm.kv_shead = kv_shead;
    prm.bt = block_tables;
    prm.bt_sb = bt_sb;
    prm.max_blocks = max_blocks;
    prm.seq_lens = seq_lens;
    prm.B = B;
    prm.Hkv = Hkv;
    prm.vg = 1;
    prm.num_pool_blocks = num_pool_blocks;
    prm.err = sink;
    hipStream_t st = as_stream(stream);
    if (mode == 0) {
        // The decode kernel's default partition: one round of 2048 waves (or the range floor).
        prm.workers = pa::resolve_workers(0, B, Hkv, max_blocks, block_size);
        prm.wg_waves = pa::kWaves;
        const int blocks = (int)ceil_div(prm.workers, pa::kWaves);
        if (D == 128)
            hipLaunchKernelGGL((pa::decode_split_kernel<128, 16, 1, true, false, true>), dim3(blocks),
                               dim3(pa::kWaves * 64), 0, st, prm);
        else
            hipLaunchKernelGGL((pa::decode_split_kernel<64, 16, 1, true, false, true>), dim3(blocks),
                               dim3(pa::kWaves * 64), 0, st, prm);
    } else {
        const int groups = pa::kDefaultWorkers / Hkv;
        if (D == 128)
            hipLaunchKernelGGL((pa::kv_block_probe_kernel<128>), dim3(groups), dim3(64 * Hkv), 0, st, prm);
        else
            hipLaunchKernelGGL((pa::kv_block_probe_kernel<64>), dim3(groups), dim3(64 * Hkv), 0, st, prm);
    }
    return check_launch(what);
}
