// Weight-only int8 linear (W8A16) for gfx950: quantize, tile pack, and the
// fused-dequant GEMV (VALU, small M) / GEMM (MFMA) kernels.
//
// Replaces the reference's quantized-linear slot (autoawq WQLinear, loaded at
// runtime/phase2/worker_server.py:194-205) with a build-defined int8 format:
// per-output-channel symmetric absmax int8 weights, fp16 scales.
//
// Packed layout (also restated in oracle/int8_quant.py): tiles of 16 rows x 64
// columns (1 KiB), k-major: tile (nt, kt) is at byte (kt*NT + nt)*1024, NT = N/16.
// In a tile, lane l = 16*g + r owns 16 bytes at 16*l: row nt*16 + r, columns
// kt*64 + 16*g + [0, 16). One wave streams a whole tile with one coalesced
// 128-bit load per lane, and waves that own neighbouring n-tiles and step
// through k together sweep one contiguous window of the weights: measured on
// MI355X over the 117 MB gate||up matrix, 6.1 TB/s against 4.3 TB/s when each
// n-tile's K run is contiguous instead (1792 scattered 1 KiB streams). Stored bytes are q ^ 0x80, so that
// fp16(0x6400 | byte) = 1024 + q + 128 and one packed fp16 add of -1152
// recovers q exactly: the dequant is 2 v_perm_b32 + 2 v_pk_add_f16 per 4 weights.
//
// Work split of the VALU GEMV (M <= 4): a workgroup owns NPW n-tiles (16*NPW
// output channels) for the whole K; its waves take interleaved k-tiles (wave w:
// w, w+WAVES, ...) so concurrent waves read adjacent kilobytes; partial sums
// meet in LDS. The MFMA GEMM (M > 4) splits the other way, see gemm_mfma_kernel.
// Both apply the per-channel scale and the bias once, in the epilogue.
#include "common.h"
#include "w8a16_tiles.h"

namespace mx {
namespace w8a16 {

// ---------------------------------------------------------------------------
// Quantize: one workgroup of 256 threads per output channel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ w, int64_t K, int8_t* __restrict__ q,
                                                       uint16_t* __restrict__ scale) {
    const int64_t row = blockIdx.x;
    const float* wr = w + row * K;
    float amax = 0.0f;
    int bad = 0;
    for (int64_t j = threadIdx.x; j < K; j += 256) {
        const float a = fabsf(wr[j]);
        bad |= !(a <= 3.4028235e38f);  // NaN or inf
        amax = fmaxf(amax, a);
    }
    for (int off = 32; off > 0; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off));
        bad |= __shfl_xor(bad, off);
    }
    __shared__ float s_max[4];
    __shared__ int s_bad[4];
    if ((threadIdx.x & 63) == 0) {
        s_max[threadIdx.x >> 6] = amax;
        s_bad[threadIdx.x >> 6] = bad;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    bad = s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3];
    // IEEE division (the library is built with correctly rounded fp32 divide).
    const float s32 = fminf(amax / 127.0f, 65504.0f);
    _Float16 sh = (_Float16)s32;
    if (amax == 0.0f) {
        sh = (_Float16)1.0f;
    } else if (sh == (_Float16)0.0f) {
        sh = __builtin_bit_cast(_Float16, (uint16_t)0x0001);
    }
    if (bad) sh = __builtin_bit_cast(_Float16, (uint16_t)0x7e00);  // NaN scale flags a non-finite row
    if (threadIdx.x == 0) scale[row] = __builtin_bit_cast(uint16_t, sh);
    const float sf = (float)sh;
    for (int64_t j = threadIdx.x; j < K; j += 256) {
        float v = __builtin_rintf(wr[j] / sf);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[row * K + j] = bad ? (int8_t)0 : (int8_t)(int)v;
    }
}

// ---------------------------------------------------------------------------
// Pack: one thread per 16-byte lane slot of the tile layout.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_kernel(const int8_t* __restrict__ q, int64_t K, int64_t KT, int64_t slots,
                                                   uint8_t* __restrict__ packed) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= slots) return;
    const int64_t tile = idx >> 6;
    const int lane = (int)(idx & 63);
    const int64_t NT = slots / (64 * KT);
    const int64_t kt = tile / NT, nt = tile % NT;
    const int r = lane & 15, g = lane >> 4;
    const uint4 src = *reinterpret_cast<const uint4*>(q + (nt * kTileN + r) * K + kt * kTileK + g * 16);
    const uint32_t flip = 0x80808080u;
    const uint4 dst{src.x ^ flip, src.y ^ flip, src.z ^ flip, src.w ^ flip};
    *reinterpret_cast<uint4*>(packed + idx * 16) = dst;
}

template <int NPW, int XV>
struct Stage {
    uint4 w[NPW];
    half8v x[XV];
};

// GEMV on the VALU for small M (v_dot2_f32_f16 against exact fp16 weights).
// GU: the gate||up projection with SwiGLU in the epilogue (interleaved rows, as the MFMA
// kernel's GU): the pair of rows r and r + 8 of an n-tile are gate and up channel
// 8*nt + r; y is [M, N/2] and receives fp16(fp16(silu(g)) * u) with g and u rounded to
// fp16 exactly as this kernel's plain epilogue rounds them. This covers gate||up shapes
// whose MFMA launch would split K (the Qwen2-0.5B MLP) at M <= 4.
template <int M, int WAVES, int P, bool GU = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_valu_kernel(const uint16_t* __restrict__ x, int64_t xs,
                                                               const uint8_t* __restrict__ w,
                                                               const uint16_t* __restrict__ scale,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ y, int64_t ys, int KT) {
    const int nt = blockIdx.x, NT = gridDim.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r = lane & 15;
    const uint4* wbase = reinterpret_cast<const uint4*>(w) + (int64_t)nt * 64;  // tile (nt, kt): + kt*NT*64
    const _Float16* xbase = reinterpret_cast<const _Float16*>(x);
    const int nj = wave < KT ? (KT - wave + WAVES - 1) / WAVES : 0;
    int xoff[M];
#pragma unroll
    for (int m = 0; m < M; ++m) xoff[m] = (int)(m * xs) + g * 16;

    auto load = [&](int j, Stage<1, 2 * M>& st) {
        const int kt = wave + (j < nj ? j : nj - 1) * WAVES;
        st.w[0] = load_wtile(wbase + (int64_t)kt * NT * 64 + lane);
        const _Float16* xk = xbase + kt * kTileK;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            st.x[2 * m] = load_half8(xk + xoff[m]);
            st.x[2 * m + 1] = load_half8(xk + xoff[m] + 8);
        }
    };
    auto compute = [&](const Stage<1, 2 * M>& st, float (&acc)[M]) {
        const half8v w0 = dequant8(st.w[0].x, st.w[0].y);
        const half8v w1 = dequant8(st.w[0].z, st.w[0].w);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            acc[m] = dot8(st.x[2 * m], w0, acc[m]);
            acc[m] = dot8(st.x[2 * m + 1], w1, acc[m]);
        }
    };

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    if (nj > 0) {
        Stage<1, 2 * M> st[P];
        PIPELINE_BODY(P, nj, st, load, compute(st[s], acc))
    }
    // Lanes r, r+16, r+32, r+48 hold the four 16-column slices of row r.
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = xor_sum_16_32(acc[m]);
    __shared__ float red[WAVES][M][kTileN];
    if (g == 0) {
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][m][r] = acc[m];
    }
    __syncthreads();
    // M * kTileN <= 64 threads: all in wave 0, so the GU lane swap below stays in one wave.
    if (threadIdx.x < M * kTileN) {
        const int m = threadIdx.x / kTileN, rr = threadIdx.x % kTileN;
        float s = 0.0f;
#pragma unroll
        for (int wv = 0; wv < WAVES; ++wv) s += red[wv][m][rr];
        const int64_t n = (int64_t)nt * kTileN + rr;
        float v = s * h2f(scale, n);
        if (bias) v += h2f(bias, n);
        if constexpr (!GU) {
            y[m * ys + n] = f2h_bits(v);
        } else {
            const float vh = (float)(_Float16)pin_f32(v);  // this lane's projection as fp16
            const float other = __shfl_xor(vh, 8);         // lane rr ^ 8: the matching up channel
            if (rr < 8) {
                const _Float16 sg = (_Float16)silu_f32(vh);
                y[m * ys + (int64_t)nt * (kTileN / 2) + rr] = f2h_bits((float)sg * other);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM on MFMA (v_mfma_f32_16x16x32_f16): A = x rows (16 per m-tile), B =
// dequantized weight tile (16 output channels), C = y^T slice. Lane l feeds A
// row l%16 / B column l%16 with the 8 k-values 16*(l/16) + 8*j + [0, 8) of the
// tile for MFMA j in {0, 1}; A and B use the same k-assignment, so any k order
// the instruction applies is consistent. C element i of lane l is row
// 4*(l/16) + i, column l%16.
//
// Work split: the WAVES waves of a workgroup own different n-tiles (wave w:
// tiles (blockIdx.x*WAVES + w)*NPW + [0, NPW)) and walk the same k-tiles of the
// workgroup's K split (blockIdx.y of gridDim.y) in step. Every k-tile of x
// ([16*MT rows x 64] fp16) is fetched once per workgroup with coalesced
// 16-byte loads, written to a padded LDS double buffer, and read back as MFMA
// fragments by all waves after one barrier. Loading the fragments straight
// from global memory instead (each 16-byte lane load touching 16 x rows)
// made the x reads, not the weight stream, the limit: at M=32 every wave
// pulled 4 bytes of x per byte of weights through L1.
//
// A wave owns whole output tiles, so there is no cross-wave reduction. With one
// split, the epilogue writes fp16 y (scale, bias); otherwise it writes the
// scaled fp32 partial of its split, which the caller or reduce_kernel adds.
// ---------------------------------------------------------------------------
// SW: x is the SwiGLU product of a gate||up row, silu(gate[k]) * up[k], formed while
// staging each x k-tile: `x` points at gate_up rows [M, 2K] (gate in columns [0, K),
// up in [K, 2K), row stride xs), rounded as the unfused path rounds it
// (fp16(fp16(silu(g)) * u), mx_silu_mul).
//
// GU: gate||up output with the SwiGLU product taken in the epilogue. The weight rows
// are interleaved in groups of 8 (rows 16t + [0, 8) are gate channels 8t + [0, 8),
// rows 16t + [8, 16) the matching up channels; see mx_w8a16_gateup_interleave), so
// the lanes holding gate channel c and up channel c differ by 8 and one lane swap
// pairs them. y is [M, N/2] and receives fp16(fp16(silu(g)) * u), g and u rounded to
// fp16 first as the unfused gate/up projections are. Needs one K split.
//
// KW > 1 (split partials only): the workgroup's waves form KW groups of WAVES / KW that
// walk the KW equal parts of the split's k-range side by side, each with its own x
// staging; their accumulators are summed in LDS (part 0 first) before the one partial of
// the split is written. The host requires KT % (KS * KW) == 0, so every group takes the
// same number of steps and meets every barrier.
//
// MW > 1: the waves of a k part also split the rows: wave (mw, wn) computes m-tiles
// mw*MT .. mw*MT + MT - 1 of the MW*MT staged (MW*MT*16 x rows per k-tile) for its NPW
// n-tiles, so MT counts m-tiles per wave and the MW waves of one wn read the same weight
// tiles (the repeats hit L2).
// Waves per SIMD the NPW = 1, MT <= 2 instances without k parts must fit: left free the
// compiler uses 226 VGPRs (2 waves per SIMD), so a 768-workgroup launch (qkv at M=32) ran in
// 1.5 rounds; at 3 it takes 166 VGPRs without spills and one round (qkv 12.5 -> 10.3 us on
// MI355X). The gate||up SwiGLU instance (7 waves, one workgroup per CU) fits either way, yet
// its 166-VGPR schedule streams faster: 26.5-28.0 -> 24.3-24.4 us at M=32 in the decode step.
// The k-part instances (o, down) measured the same at 166 and 226 and stay unbounded.
#ifndef MX_GEMM_MIN_WAVES
#define MX_GEMM_MIN_WAVES 3
#endif
// NJX > 0: the k part's whole x range (at most NJX k-tiles) is staged in LDS once, its loads issued
// before the pipeline's weight loads and stored after them, with one barrier; the main loop then
// reads fragments at the k-tile's column offset and meets no barrier. Results are identical to the
// per-k-tile staging. Measured on MI355X: a barrier per k-tile cost the Qwen2-0.5B step (k ranges
// of 5-14 tiles) about 9 % of its time.
//
// The body takes its workgroup's grid coordinates (gx, ks) and the split count KS as arguments, so
// that the fused MLP launch (mlp_fused_kernel) can run it twice. FUSE: 0 a plain launch; 1 the
// gate||up phase of the fused launch, whose SwiGLU outputs are stored as whole lines written through
// the XCD's L2 (sc1), so that workgroups on the other XCDs can read them in the same launch; 2 its
// down phase, which issues its first P stages of weight loads, waits for the activations of its k
// range (mlp_wait) and then reads them.
struct MlpWait {
    int* sync = nullptr;  // per-chunk arrival counters, then kMlpDone and kMlpErr
    int chunk_ch = 0;     // activation channels per chunk: one k part of one split of down
    int group_ch = 0;     // activation channels per gate||up workgroup
    int groups = 0;       // gate||up workgroups
};
constexpr int kMlpMaxChunks = 32, kMlpDone = 32, kMlpErr = 33, kMlpSyncWords = 64;
// Polls of the arrival counter before a wait gives up (each a device-coherent load of about a
// microsecond plus a short sleep): a wait that should last tens of microseconds ends after tens of
// milliseconds at most, sets kMlpErr bit 1 and goes on with whatever the activations hold.
constexpr int kMlpSpinLimit = 1 << 15;

// Gate||up workgroups whose activation channels overlap chunk c.
__device__ __forceinline__ int mlp_chunk_arrivals(const MlpWait& wt, int c) {
    const int lo = c * wt.chunk_ch / wt.group_ch;
    int hi = ((c + 1) * wt.chunk_ch - 1) / wt.group_ch;
    if (hi > wt.groups - 1) hi = wt.groups - 1;
    return hi - lo + 1;
}

// Thread 0 waits until every gate||up workgroup that writes the chunks of k parts [0, KW) of split
// ks has arrived; the workgroup's barrier then releases every wave.
template <int KW>
__device__ __forceinline__ void mlp_wait(const MlpWait& wt, int ks) {
    if (threadIdx.x == 0) {
        for (int kw = 0; kw < KW; ++kw) {
            const int c = ks * KW + kw;
            const int want = mlp_chunk_arrivals(wt, c);
            int polls = 0;
            while (__hip_atomic_load(wt.sync + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want) {
                if (++polls > kMlpSpinLimit) {
                    atomicOr(wt.sync + kMlpErr, 1);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
    }
    __syncthreads();
}

template <int MT, int NPW, int WAVES, int P, bool SW, bool GU, int KW, int MW, int NJX, int FUSE>
__device__ __forceinline__ void gemm_body(const int gx, const int ks, const int KS, const uint16_t* __restrict__ x,
                                          int64_t xs, int M, const uint8_t* __restrict__ w,
                                          const uint16_t* __restrict__ scale, const uint16_t* __restrict__ bias,
                                          uint16_t* __restrict__ y, int64_t ys, int KT, int NT,
                                          float* __restrict__ partial, const MlpWait& wt) {
    static_assert(FUSE == 0 || (NJX == 0 && !SW && MW == 1 && NPW == 1), "fused phases: plain 1-n-tile shapes");
    static_assert(FUSE != 1 || GU, "the fused gate||up phase has the SwiGLU epilogue");
    static_assert(FUSE != 2 || !GU, "the fused down phase writes partials");
    constexpr int ROWS = MW * MT * 16;  // x rows staged per k-tile (MW waves along M, MT m-tiles each)
    constexpr int RS = kTileK + 8;  // LDS row stride (halfs): 144 bytes, rows start 4 banks apart
    constexpr int WN = WAVES / (KW * MW);  // waves along N per k part, each owning NPW n-tiles
    constexpr int WP = WN * MW;            // waves per k part
    static_assert(WN * KW * MW == WAVES, "waves: k parts x m groups x n groups");
    constexpr int XCH = ROWS * 8;   // 16-byte chunks of one x k-tile
    constexpr int XC = (XCH + WP * 64 - 1) / (WP * 64);
    static_assert(NJX == 0 || (!SW && MW == 1), "whole-range x staging: plain x, one m group");
    constexpr int RSX = NJX * kTileK + 8;  // row stride (halfs) of a whole-range buffer: rows 4 banks apart
    constexpr int XF = NJX > 0 ? (ROWS * NJX * 8 + WP * 64 - 1) / (WP * 64) : 1;  // chunks per thread
    __shared__ __attribute__((aligned(16))) _Float16 xl[KW][NJX > 0 ? 1 : 2][NJX > 0 ? ROWS * RSX : ROWS * RS];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave / WP, wm = wave - kw * WP;
    const int mw = wm / WN, wn = wm - mw * WN;
    const int kt_split = (int)((int64_t)ks * KT / KS);
    const int nj = ((int)((int64_t)(ks + 1) * KT / KS) - kt_split) / KW;
    const int kt_lo = kt_split + kw * nj;
    const int ltid = tid - kw * WP * 64;  // thread index within the k part
    const int lane = tid & 63;
    const int g = lane >> 4, r = lane & 15;
    const int nt_w = (gx * WN + wn) * NPW;
    const bool valid = nt_w < NT;                 // NT % NPW == 0: a wave is all in or all out
    const int nt_c = valid ? nt_w : NT - NPW;     // out-of-range waves load (and drop) the last tiles
    const uint4* wbase = reinterpret_cast<const uint4*>(w) + (int64_t)nt_c * 64;  // tile (nt_c + p, kt): + (kt*NT + p)*64

    // x chunks of this thread: chunk c = ltid + u*WP*64 (wrapped when the tile has
    // fewer chunks than threads; the duplicate writes store identical bytes).
    int xsrc[XC], xdst[XC];
#pragma unroll
    for (int u = 0; u < XC; ++u) {
        const int c = (ltid + u * WP * 64) % XCH;
        const int row = c / 8, col = (c % 8) * 8;
        const int rc = row < M ? row : M - 1;
        xsrc[u] = (int)(rc * xs) + col;
        xdst[u] = row * RS + col;
    }
    const _Float16* xbase = reinterpret_cast<const _Float16*>(x);

    struct St {
        uint4 w[NPW];
        uint4 x[XC];
        uint4 up[SW ? XC : 1];
    };
    const int up_off = KT * kTileK;  // SW: the up half of a gate_up row
    auto load_w = [&](int j, St& st) {
        const int kt = kt_lo + (j < nj ? j : nj - 1);
#pragma unroll
        for (int p = 0; p < NPW; ++p) st.w[p] = load_wtile<MW == 1>(wbase + ((int64_t)kt * NT + p) * 64 + lane);
    };
    auto load_x = [&](int j, St& st) {
        const int kt = kt_lo + (j < nj ? j : nj - 1);
        if constexpr (NJX == 0) {
#pragma unroll
            for (int u = 0; u < XC; ++u) {
                // FUSE == 2: plain loads of activations written in this launch. Each line of them has
                // one writer, which wrote it through to memory before counting itself, and no cache of
                // this CU or XCD holds it before its chunk's wait ends (caches start the launch clean and
                // nothing reads the activations earlier), so the first load fetches the final line.
                st.x[u] = *reinterpret_cast<const uint4*>(xbase + xsrc[u] + kt * kTileK);
                if (SW) st.up[u] = *reinterpret_cast<const uint4*>(xbase + xsrc[u] + up_off + kt * kTileK);
            }
        }
    };
    auto load = [&](int j, St& st) {
        load_w(j, st);
        load_x(j, st);
    };
    // NJX: chunk c = ltid + u * WP * 64 of the part's ROWS x (nj * 64) range (rows past M read row
    // M - 1; chunks past the range load chunk 0 and are stored to row 0's padding, which no fragment
    // read touches). Stores are unconditional and a scheduling barrier keeps these loads ahead of
    // the pipeline's weight loads: waiting for them then never waits for the weights (loads
    // complete in order). Sunk into conditional stores, they made the compiler drain every weight
    // load before the first MFMA.
    uint4 xf[XF];
    int xfo[XF];
    if constexpr (NJX > 0) {
        const int cpr = nj * 8;  // chunks per row
#pragma unroll
        for (int u = 0; u < XF; ++u) {
            const int c = ltid + u * WP * 64;
            const bool in = c < ROWS * cpr;
            const int cc = in ? c : 0;
            const int row = cc / cpr, col = (cc - row * cpr) * 8;
            const int rc = row < M ? row : M - 1;
            xf[u] = *reinterpret_cast<const uint4*>(xbase + (int64_t)rc * xs + (int64_t)kt_lo * kTileK + col);
            xfo[u] = in ? row * RSX + col : NJX * kTileK;
        }
        asm volatile("" ::: "memory");  // no load moves across: x first, then the weights
    }

    float4v acc[NPW][MT];
#pragma unroll
    for (int p = 0; p < NPW; ++p)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[p][mt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // Buffer parity alternates per k-tile. Buffer b is rewritten two k-tiles after
    // it was read; every wave finished that read before the barrier in between.
    int step = 0;
    auto compute = [&](const St& st) {
        const _Float16* frag = &xl[kw][0][0] + step * kTileK;  // NJX: this k-tile's columns
        constexpr int FRS = NJX > 0 ? RSX : RS;
        if constexpr (NJX == 0) {
        _Float16* buf = xl[kw][step & 1];
        frag = buf;
#pragma unroll
        for (int u = 0; u < XC; ++u) {
            if (SW) {
                const half8v gt = __builtin_bit_cast(half8v, st.x[u]);
                const half8v up = __builtin_bit_cast(half8v, st.up[u]);
                half8v a;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const _Float16 sg = (_Float16)silu_f32((float)gt[e]);
                    a[e] = (_Float16)((float)sg * (float)up[e]);
                }
                *reinterpret_cast<uint4*>(buf + xdst[u]) = __builtin_bit_cast(uint4, a);
            } else {
                *reinterpret_cast<uint4*>(buf + xdst[u]) = st.x[u];
            }
        }
        __syncthreads();
        }
        half8v a[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const _Float16* src = frag + ((mw * MT + mt) * 16 + r) * FRS + 16 * g;
            a[mt][0] = __builtin_bit_cast(half8v, *reinterpret_cast<const uint4*>(src));
            a[mt][1] = __builtin_bit_cast(half8v, *reinterpret_cast<const uint4*>(src + 8));
        }
#pragma unroll
        for (int p = 0; p < NPW; ++p) {
            const half8v b0 = dequant8(st.w[p].x, st.w[p].y);
            const half8v b1 = dequant8(st.w[p].z, st.w[p].w);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[p][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][0], b0, acc[p][mt], 0, 0, 0);
                acc[p][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][1], b1, acc[p][mt], 0, 0, 0);
            }
        }
        ++step;
    };
    // The epilogue's per-channel scale and bias are loaded right after the pipeline's first
    // stages, so their round trip overlaps the main loop instead of following it (measured
    // 0.4-0.9 us per wave between the last k-tile and the stores when loaded in the epilogue).
    // Out-of-range waves load the clamped tiles' values and store nothing.
    // - One n-tile or one m-tile per wave, not SwiGLU: converted to fp32 where they are loaded.
    // - NJX instances, the gate||up SwiGLU ones and the wide ones of at most two m-tiles and four
    //   n-tiles: loaded raw (16-bit values held through the loop) and converted after the MFMAs,
    //   behind a scheduling barrier. Converted where they were loaded, the conversion (and so a
    //   wait for the loads, which follow the first stages in the queue) went to the loop's start;
    //   held as fp32 they made the SwiGLU instances spill.
    // - The other wide instances (two n-tiles at two m-tiles, three or more m-tiles), which are at
    //   or past their register budget, load them in the epilogue.
    constexpr bool kFloatEarly = !GU && (NPW == 1 || MT == 1);
    constexpr bool kRaw = NJX > 0 || (!kFloatEarly && (NPW == 1 || (MT <= 2 && NPW == 4)));
    constexpr bool kEarly = kFloatEarly || kRaw;
    float sc_pre[NPW], bi_pre[NPW];
    uint16_t sc_raw[NPW], bi_raw[NPW];
    auto convert_epilogue = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        const bool with_bias = KS == 1 && bias;
#pragma unroll
        for (int p = 0; p < NPW; ++p) {
            sc_pre[p] = (float)__builtin_bit_cast(_Float16, sc_raw[p]);
            bi_pre[p] = with_bias ? (float)__builtin_bit_cast(_Float16, bi_raw[p]) : 0.0f;
        }
    };
    auto load_epilogue = [&]() {
        if constexpr (!kEarly) return;
#pragma unroll
        for (int p = 0; p < NPW; ++p) {
            const int64_t n = (int64_t)(nt_c + p) * kTileN + r;
            if constexpr (kRaw) {  // unconditional loads (no bias: read the scale, use 0)
                sc_raw[p] = scale[n];
                bi_raw[p] = ((KS == 1 && bias) ? bias : scale)[n];
            } else {
                sc_pre[p] = h2f(scale, n);
                bi_pre[p] = (KS == 1 && bias) ? h2f(bias, n) : 0.0f;
            }
        }
    };
    // NJX: the whole-range x reaches LDS after the pipeline's first weight loads are issued. The
    // stores are written inline (not in a lambda): captured by reference, xf went to scratch memory.
#define MX_NJX_HOOK                                                                       \
    load_epilogue();                                                                      \
    if constexpr (NJX > 0) {                                                              \
        _Pragma("unroll") for (int u = 0; u < XF; ++u)                                    \
            *reinterpret_cast<uint4*>(&xl[kw][0][0] + xfo[u]) = xf[u];                    \
        __syncthreads();                                                                  \
    }
    if (nj > 0) {
        if constexpr (NJX > 0) {
            // Every k-tile of the range in flight at once (nj <= NJX) and the compute unrolled: no
            // loop-carried stages, whose register copies at the loop entry made the first MFMA wait
            // for every load of the pipeline's first round.
            St st[NJX];
#pragma unroll
            for (int j = 0; j < NJX; ++j)
                if (j < nj) load(j, st[j]);
            MX_NJX_HOOK
#pragma unroll
            for (int j = 0; j < NJX; ++j)
                if (j < nj) compute(st[j]);
        } else {
            St st[P];
            if constexpr (FUSE == 2) {
                // The first stages' weights go out before the wait, their activations after it.
#pragma unroll
                for (int s = 0; s < P; ++s) load_w(s, st[s]);
                mlp_wait<KW>(wt, ks);
#pragma unroll
                for (int s = 0; s < P; ++s) load_x(s, st[s]);
                MX_NJX_HOOK
                PIPELINE_REST(P, nj, st, load, compute(st[s]))
            } else {
                PIPELINE_BODY_HOOK(P, nj, st, load, compute(st[s]), MX_NJX_HOOK)
            }
        }
    } else {
        load_epilogue();
    }
    if constexpr (kRaw) convert_epilogue();
#undef MX_NJX_HOOK
    const int N = NT * kTileN;
    if constexpr (KW > 1) {
        // Parts 1.. hand their accumulators to part 0 through LDS; every wave reaches this
        // barrier (out-of-range waves too) before any of them leaves.
        __shared__ float4v red[KW - 1][WP][NPW][MT][64];
        if (kw > 0) {
#pragma unroll
            for (int p = 0; p < NPW; ++p)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) red[kw - 1][wm][p][mt][lane] = acc[p][mt];
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int q = 0; q < KW - 1; ++q)
#pragma unroll
            for (int p = 0; p < NPW; ++p)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) acc[p][mt] += red[q][wm][p][mt][lane];
    }
    if (GU) {
        // FUSE == 1: the workgroup's [ROWS, 64] activation tile is gathered in LDS first and stored
        // as whole 128-byte lines of each row (write-through, see below).
        __shared__ __attribute__((aligned(16))) uint16_t act_tile[FUSE == 1 ? ROWS : 1][FUSE == 1 ? WN * 8 : 1];
        // Every lane takes part in the swap; out-of-range waves just do not store.
#pragma unroll
        for (int p = 0; p < NPW; ++p) {
            const int c = (nt_c + p) * (kTileN / 2) + (r & 7);  // SwiGLU channel of this lane pair
            const int64_t n = (int64_t)(nt_c + p) * kTileN + r;
            const float sc = kEarly ? sc_pre[p] : h2f(scale, n);
            const float bi = kEarly ? bi_pre[p] : (bias ? h2f(bias, n) : 0.0f);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = (float)(_Float16)pin_f32(acc[p][mt][i] * sc + bi);  // this lane's projection
                    const float other = __shfl_xor(v, 8);
                    const int m = (mw * MT + mt) * 16 + 4 * g + i;
                    if (valid && r < 8 && m < M) {
                        const _Float16 sg = (_Float16)silu_f32(v);
                        if constexpr (FUSE == 1)
                            act_tile[m][wn * 8 + (r & 7)] = f2h_bits((float)sg * other);
                        else
                            y[(int64_t)m * ys + c] = f2h_bits((float)sg * other);
                    }
                }
        }
        if constexpr (FUSE == 1) {
            // 16 threads per row, 8 bytes each: every store instruction covers whole lines. The
            // stores are device-coherent (sc1, written through the XCD's L2), so that a workgroup on
            // another XCD that waits for this one's arrival reads them from memory; the group's
            // channels are whole lines of each row (the caller checks the alignment), so no line of
            // the activations is written from two XCDs.
            static_assert(FUSE != 1 || (WN * 8 * 2 == 128 && ROWS * 16 <= WAVES * 64), "one line per row, one store each");
            __syncthreads();
            const int row = tid >> 4, q = tid & 15;
            if (row < ROWS && row < M && nt_w - wn * NPW < NT) {
                const uint64_t v = *reinterpret_cast<const uint64_t*>(&act_tile[row][q * 4]);
                __hip_atomic_store(reinterpret_cast<uint64_t*>(y + (int64_t)row * ys + (int64_t)gx * WN * 8) + q, v,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return;
    }
    if (!valid) return;
#pragma unroll
    for (int p = 0; p < NPW; ++p) {
        const int64_t n = (int64_t)(nt_w + p) * kTileN + r;
        const float sc = kEarly ? sc_pre[p] : h2f(scale, n);
        const float bi = kEarly ? bi_pre[p] : ((KS == 1 && bias) ? h2f(bias, n) : 0.0f);  // 0 unless unsplit
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = (mw * MT + mt) * 16 + 4 * g + i;
                if (m >= M) continue;
                if (KS == 1) y[(int64_t)m * ys + n] = f2h_bits(pin_f32(acc[p][mt][i] * sc + bi));
                else partial[((int64_t)ks * M + m) * N + n] = acc[p][mt][i] * sc;
            }
    }
}

template <int MT, int NPW, int WAVES, int P, bool SW = false, bool GU = false, int KW = 1, int MW = 1, int NJX = 0>
__global__ __launch_bounds__(WAVES * 64, (NPW == 1 && !SW && MT <= 2 && KW == 1 && MW == 1) ? MX_GEMM_MIN_WAVES : 1) void gemm_mfma_kernel(const uint16_t* __restrict__ x, int64_t xs, int M,
                                                               const uint8_t* __restrict__ w,
                                                               const uint16_t* __restrict__ scale,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ y, int64_t ys, int KT, int NT,
                                                               float* __restrict__ partial) {
    gemm_body<MT, NPW, WAVES, P, SW, GU, KW, MW, NJX, 0>(blockIdx.x, blockIdx.y, gridDim.y, x, xs, M, w, scale, bias, y,
                                                         ys, KT, NT, partial, MlpWait{});
}

// y[m, n] = fp16(bias[n] + the splits' partial[ks][m][n] in split order), one fp32 add each. A
// thread owns 8 consecutive outputs (N % 16 == 0). KS > 0 is the split count known at compile time:
// every split's two 16-byte loads go out before the first add, one memory round trip in all; KS == 0
// loops over `splits`. A runtime loop of one element per thread made the compiler wait for each
// split's load before issuing the next: one round trip per split.
template <int KS>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ partial, int splits, int M, int N,
                                                     const uint16_t* __restrict__ bias, uint16_t* __restrict__ y,
                                                     int64_t ys) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int G8 = N / 8;
    if (idx >= (int64_t)M * G8) return;
    const int m = (int)(idx / G8), n = (int)(idx % G8) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bias ? h2f(bias, n + e) : 0.0f;
    const float* p = partial + (int64_t)m * N + n;
    const int64_t stride = (int64_t)M * N;
    if constexpr (KS > 0) {
        float4v a[KS][2];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            a[k][0] = *reinterpret_cast<const float4v*>(p + k * stride);
            a[k][1] = *reinterpret_cast<const float4v*>(p + k * stride + 4);
        }
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] += a[k][e / 4][e % 4];
    } else {
        for (int k = 0; k < splits; ++k) {
            const float4v a0 = *reinterpret_cast<const float4v*>(p + k * stride);
            const float4v a1 = *reinterpret_cast<const float4v*>(p + k * stride + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] += a0[e];
                v[4 + e] += a1[e];
            }
        }
    }
    uint16_t* yr = y + (int64_t)m * ys + n;
    if ((reinterpret_cast<uintptr_t>(yr) & 15) == 0) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (uint32_t)f2h_bits(pin_f32(v[2 * e])) | ((uint32_t)f2h_bits(pin_f32(v[2 * e + 1])) << 16);
        *reinterpret_cast<uint4*>(yr) = uint4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) yr[e] = f2h_bits(pin_f32(v[e]));
    }
}

// Largest M handled by the VALU GEMV; above it the MFMA kernel runs.
constexpr int kValuMaxM = 4;
constexpr int kMaxRows = 128;  // rows per MFMA launch (8 m-tiles); larger M runs in chunks
// Waves per GEMV workgroup (one workgroup per n-tile, the waves taking interleaved k-tiles): 4
// where the grid alone covers the chip (more than 256 n-tiles) or K is short or long (at most 32
// or at least 128 k-tiles), else 8 (few workgroups that must each pull a middling K: the
// Qwen2-0.5B down projection, 56 n-tiles x 76 k-tiles). 16 spilled. Measured on MI355X, 40-50
// distinct weight copies per graph, 8 -> 4 waves, M = 1..4: Llama-3-8B qkv 9.4-15.9 ->
// 8.5-14.4 us, down 16.0-23.8 -> 14.0-23.5 us; Qwen2-0.5B qkv 3.8-4.6 -> 3.2-3.9 us, o 3.7-4.5 ->
// 3.2-3.9 us, gate||up (9728 x 896) 9.0-11.8 -> 5.5-7.5 us; the Llama o / config-1 shape (256 x 64
// tiles) 6.1-9.0 either way, 7.5 against 8.1 us at M = 2, so it keeps 8.
static int gemv_waves(int NT, int KT) { return (NT > 256 || KT <= 32 || KT >= 128) ? 4 : 8; }
constexpr int kMfmaWaves = 4;
constexpr int kWideGrid = 256;    // at least this many n-groups: no K split
constexpr int kSplitGrid = 512;   // otherwise split K until the grid reaches this many workgroups
constexpr int kMaxSplits = 16;
// k-tiles per K range at least: 1 for the plain split, 4 for the M-split shape (below). Ranges of
// one or two k-tiles let the short-K projections spread over more workgroups: the Qwen2-0.5B o
// (896 x 896, 14 k-tiles) at 16 rows went from 2 to 8 ranges, 4.1 -> 3.5 us per launch and the
// config-3 step 0.958 -> 0.950 ms (MI355X, two interleaved rounds). The Llama-3-8B shapes reach the
// grid bound first and keep their ranges.
constexpr int kMinSplitTiles = 1;
constexpr int kMinBigSplitTiles = 4;

// Pipeline depth from the VGPRs one stage costs (4 per 1 KiB weight tile, 8
// per x row fragment of 32 bytes) after the accumulators.
// GEMV pipeline depth per M (a stage holds 4 VGPRs of weights and 8 per x row); at M = 2
// a depth of 8 reached 256 VGPRs and spilled.
constexpr int gemv_depth(int M) { return M <= 1 ? 8 : (M == 2 ? 6 : (M == 3 ? 5 : 4)); }
#ifndef MX_GEMM_DEPTH_SMALL_M
#define MX_GEMM_DEPTH_SMALL_M 8
#endif
constexpr int mfma_depth(int MT) { return MT <= 2 ? MX_GEMM_DEPTH_SMALL_M : (MT <= 4 ? 6 : 4); }

// m-tiles of a chunk of M rows: instantiated for 1, 2, 3, 4, 6 and 8 (5 and 7 round
// up; rows past M read row M-1 and their results are dropped).
constexpr int mt_for(int M) {
    const int mt = (M + 15) / 16;
    return mt <= 4 ? mt : (mt <= 6 ? 6 : 8);
}

// Launch plan for one chunk of at most kMaxRows rows.
struct Plan {
    bool valu;
    int MT, KS;  // KS: partials written (k ranges of the launch / KW)
    int KW;      // k parts per workgroup, summed in LDS
};

// k parts per workgroup of a split launch (M <= 64): the split's 8-wave workgroups hold
// two k parts of 4 waves each, so a launch of the same waves writes half the partials and
// their consumers read half as much (decode step at batch 32: o and down write 2 MB instead
// of 4 MB; step 4.69 -> 4.66 ms on MI355X together with the occupancy bound below).
#ifndef MX_GEMM_KPARTS
#define MX_GEMM_KPARTS 2
#endif
constexpr int kKParts = MX_GEMM_KPARTS;

// K ranges of the MFMA launch: none when the n-groups alone fill the chip, else the
// smallest power of two that gives kSplitGrid 4-wave workgroups' worth of waves (at M=32
// on the Llama-3-8B shapes: qkv, o and down 8, gate_up none). plan_for then pairs ranges
// into k parts of one workgroup where that keeps one round: o and down write 4 partials,
// qkv (384 groups of parts would need 1.5 rounds) writes 8.
static int splits_for(int NT, int KT) {
    const int groups = (NT + kMfmaWaves - 1) / kMfmaWaves;
    if (groups >= kWideGrid) return 1;
    int ks = 1;
    while (ks < kMaxSplits && groups * ks < kSplitGrid && KT / (2 * ks) >= kMinSplitTiles) ks *= 2;
    return ks;
}

// Chunks of more than 64 rows (6 or 8 m-tiles), and of 49-64 rows where use_m_split says so:
// 8-wave workgroups of 2 waves along M (each 2, 3 or 4 m-tiles, all of the chunk's rows
// staged once in LDS) by 4 along N, each
// wave holding 2 n-tiles, so every x fragment read from LDS feeds two MFMAs. The two
// m-halves read the same weight tiles (the second read is an L2 hit). With one 4-wave
// workgroup of 8 m-tiles x 1 n-tile (254 VGPRs + 48 AGPRs, one wave per SIMD) the
// Llama-3-8B projections at M = 128 ran at 1.2 TB/s (qkv 37.5, o 26.8, gate_up 75.4,
// down 44.2 us on MI355X). K is split until the grid holds about one workgroup per CU.
constexpr int kBigWaves = 8, kBigNpw = 2;
constexpr int kBigTiles = (kBigWaves / 2) * kBigNpw;  // n-tiles per workgroup
constexpr int kBigGrid = 256;
static bool big_m_shape(int NT) { return NT % kBigNpw == 0; }
static int big_splits(int NT, int KT) {
    const int groups = ceil_div(NT, kBigTiles);
    int ks = 1;
    while (ks < kMaxSplits && groups * ks * 2 <= kBigGrid && KT / (2 * ks) >= kMinBigSplitTiles) ks *= 2;
    return ks;
}

// Where the M-split shape takes a chunk: above 64 rows always (when NT is even), and at 49-64
// rows (4 m-tiles, two per wave) when its k ranges are long enough to fill its 4-deep pipeline
// several times. Measured on the Llama-3-8B shapes at M = 64 (MI355X): qkv 23.3 -> 16.5 us,
// gate_up 36.9 -> 32.7, down 24.9 -> 23.0-24.0 (k ranges of 32, 64 and 28 tiles); o, whose
// 8-tile k ranges would take two pipeline rounds, measured 14.0 -> 16.2 and keeps the 4-wave
// shape.
constexpr int kMwMinRangeTiles = 16;
static bool use_m_split(int MT, int NT, int KT) {
    if (!big_m_shape(NT)) return false;
    return MT >= 6 || (MT == 4 && KT / big_splits(NT, KT) >= kMwMinRangeTiles);
}

static Plan plan_for(int M, int NT, int KT) {
    Plan pl{};
    pl.KS = 1;
    pl.KW = 1;
    if (mt_for(M) >= 4 && use_m_split(mt_for(M), NT, KT)) {
        pl.valu = false;
        pl.MT = mt_for(M);
        pl.KS = big_splits(NT, KT);
        return pl;
    }
    // The VALU GEMV takes M <= 4 unless the n-groups alone fill the chip: there the
    // MFMA kernel's wide workgroups stream faster even with 15 padding rows (gate||up
    // at M = 1: 33.2 us GEMV, 23 us MFMA), while split shapes keep the GEMV, which needs
    // no reduce (4096 x 4096 at M = 1: 6.3 us).
    if (M <= kValuMaxM && splits_for(NT, KT) > 1) {
        pl.valu = true;
        pl.MT = M;
        return pl;
    }
    pl.valu = false;
    pl.MT = mt_for(M);
    const int ranges = splits_for(NT, KT);
    // k parts only when the launch of kKParts * 4-wave workgroups stays one round at one
    // workgroup per CU (these workgroups need more than half a CU's wave slots).
    const int groups = ceil_div(NT, kMfmaWaves);
    pl.KW = kKParts > 1 && pl.MT <= 4 && ranges % kKParts == 0 && ranges / kKParts > 1 && KT % ranges == 0 &&
                    groups * (ranges / kKParts) <= kWideGrid
                ? kKParts
                : 1;
    pl.KS = ranges / pl.KW;
    return pl;
}

static size_t workspace_for(int M, int NT, int KT) {
    const Plan pl = plan_for(M, NT, KT);
    return pl.KS > 1 ? (size_t)pl.KS * M * NT * kTileN * sizeof(float) : 0;
}

template <int M, bool GU = false>
static void launch_gemv(const uint16_t* x, int64_t xs, const uint8_t* w, const uint16_t* s, const uint16_t* b,
                        uint16_t* y, int64_t ys, int NT, int KT, hipStream_t st) {
    if (gemv_waves(NT, KT) == 4)
        hipLaunchKernelGGL((gemv_valu_kernel<M, 4, gemv_depth(M), GU>), dim3(NT), dim3(4 * 64), 0, st, x, xs, w, s, b, y,
                           ys, KT);
    else
        hipLaunchKernelGGL((gemv_valu_kernel<M, 8, gemv_depth(M), GU>), dim3(NT), dim3(8 * 64), 0, st, x, xs, w, s, b, y,
                           ys, KT);
}

template <bool GU = false>
static void launch_gemv_m(int M, const uint16_t* x, int64_t xs, const uint8_t* w, const uint16_t* s,
                          const uint16_t* b, uint16_t* y, int64_t ys, int NT, int KT, hipStream_t st) {
    switch (M) {
        case 1: launch_gemv<1, GU>(x, xs, w, s, b, y, ys, NT, KT, st); break;
        case 2: launch_gemv<2, GU>(x, xs, w, s, b, y, ys, NT, KT, st); break;
        case 3: launch_gemv<3, GU>(x, xs, w, s, b, y, ys, NT, KT, st); break;
        default: launch_gemv<4, GU>(x, xs, w, s, b, y, ys, NT, KT, st); break;
    }
}

// Workgroup shape of an unsplit launch at M <= 64: about one workgroup per CU,
// each as wide as possible, so that one x k-tile staged in LDS feeds as many
// weight tiles as possible. Every workgroup re-reads all of x: with 4-wave
// workgroups a CU loads as many x bytes as weight bytes, and those loads, not
// the weight stream, set the pace (measured on MI355X at M=32: gate_up 27.7 us
// with 448 x 4 waves, 23.3 us with 256 x 7 waves; lm_head 108.7 us with 2004 x 4
// waves, 91.3 us with 251 x 8 waves of 4 n-tiles each). The widest shape whose
// grid is one round of 240..256 workgroups wins; none: 4 waves of 1 n-tile.
struct WideShape {
    int waves, npw;
};
constexpr int kOneRoundLo = 240, kOneRoundHi = 256;
// gate||up with the SwiGLU epilogue at most this many k-tiles long (an even count, up to 32 rows,
// where no wide shape fits) runs as 8-wave workgroups of two k parts x 4 n-tiles with whole-range x
// staging, the parts summed in LDS before the epilogue: each wave's dependent chain of k-tiles is half
// as long. Measured on MI355X
// (Qwen2-0.5B gate||up, 4864 x 2 channels, 14 k-tiles, 16 rows; three interleaved rounds): 5.80-5.81 ->
// 5.36-5.39 us, the config-3 step 0.949-0.950 -> 0.941-0.942 ms. 4-wave workgroups of two k parts x 2
// n-tiles (twice the workgroups) measured no gain, 5.85-5.88 us.
constexpr int kGuShortKT = 32;
static WideShape wide_shape(int NT, bool npw1_only) {
    const WideShape cands[] = {{8, 4}, {8, 2}, {8, 1}, {7, 1}, {6, 1}, {5, 1}};
    for (const WideShape& c : cands) {
        if (c.npw > 1 && (npw1_only || NT % c.npw)) continue;
        const int groups = ceil_div(NT, c.waves * c.npw);
        if (groups >= kOneRoundLo && groups <= kOneRoundHi) return c;
    }
    return WideShape{kMfmaWaves, 1};
}

template <int MT, int NPW, int WAVES, bool SW, bool GU, int KW = 1, int MW = 1, int NJX = 0>
static void launch_shape(const uint16_t* x, int64_t xs, int M, const uint8_t* w, const uint16_t* s, const uint16_t* b,
                         uint16_t* y, int64_t ys, int NT, int KT, int KS, float* partial, hipStream_t st) {
    // Pipeline depth (k-tiles of loads in flight per wave), the deepest that fits 256 VGPRs
    // without scratch: 6 for the M-split shape spilled (24 VGPRs at 4 m-tiles), 4 fits. The wide
    // shapes (two or four n-tiles) and the SwiGLU-input instances at three or more m-tiles spilled
    // 36-216 bytes per lane at depths 4-6; at the depths below none does, and on MI355X lm_head
    // (128256 x 4096) went 99.3-102.6 -> 84.4-85.3 us at 33 rows and 100.5-103.9 -> 86.7-87.4 us at
    // 48, the SwiGLU-input down (4096 x 14336) 42.0-42.4 -> 37.5-37.7 us at 48 rows and
    // 49.1-49.5 -> 37.5-37.8 us at 64 (three interleaved pairs each).
    constexpr int P = MW > 1 ? 4
                      : NPW == 1 ? (SW && MT >= 3 ? 3 : mfma_depth(MT))
                      : NPW == 2 ? (MT == 1 ? 6 : (MT == 2 ? 4 : 3))
                                 : (MT <= 2 ? 4 : 2);
    const int groups = ceil_div(NT, (WAVES / (KW * MW)) * NPW);
    hipLaunchKernelGGL((gemm_mfma_kernel<MT, NPW, WAVES, P, SW, GU, KW, MW, NJX>), dim3(groups, KS), dim3(WAVES * 64), 0,
                       st, x, xs, M, w, s, b, y, ys, KT, NT, partial);
}

// The MFMA kernel alone: KS == 1 writes fp16 y, KS > 1 writes the scaled fp32
// partials [KS][M][N] to `partial` (no bias), each from KW k parts of its workgroups.
template <int MT, bool SW, bool GU = false>
static void launch_mfma(const uint16_t* x, int64_t xs, int M, const uint8_t* w, const uint16_t* s, const uint16_t* b,
                        uint16_t* y, int64_t ys, int NT, int KT, int KS, int KW, float* partial, hipStream_t st) {
    if constexpr (MT >= 4 && !SW) {
        if (use_m_split(MT, NT, KT)) {
            launch_shape<MT / 2, kBigNpw, kBigWaves, SW, GU, 1, 2>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);
            return;
        }
    }
    // Whole-range x staging (NJX) where a k part's range is at most 16 k-tiles and M <= 32.
    const int range = (int)ceil_div(KT, (int64_t)KS * KW);
    if constexpr (MT <= 4 && !GU && kKParts > 1) {
        if (KS > 1 && KW == kKParts) {
            if constexpr (MT <= 2 && !SW) {
                if (range <= 8) {
                    launch_shape<MT, 1, kMfmaWaves * kKParts, SW, GU, kKParts, 1, 8>(x, xs, M, w, s, b, y, ys, NT, KT, KS,
                                                                                       partial, st);
                    return;
                }
                if (range <= 16) {
                    launch_shape<MT, 1, kMfmaWaves * kKParts, SW, GU, kKParts, 1, 16>(x, xs, M, w, s, b, y, ys, NT, KT,
                                                                                        KS, partial, st);
                    return;
                }
            }
            launch_shape<MT, 1, kMfmaWaves * kKParts, SW, GU, kKParts>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);
            return;
        }
    }
    if constexpr (MT <= 4 && !SW) {
        if (KS == 1) {
            const WideShape ws = wide_shape(NT, GU);
#define MX_WIDE(W, NPW)                                                                                     \
    if (ws.waves == W && ws.npw == NPW) {                                                                   \
        launch_shape<MT, NPW, W, SW, GU>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);                \
        return;                                                                                             \
    }
            MX_WIDE(5, 1)
            MX_WIDE(6, 1)
            MX_WIDE(7, 1)
            MX_WIDE(8, 1)
            if constexpr (!GU) {
                MX_WIDE(8, 2)
                MX_WIDE(8, 4)
            }
#undef MX_WIDE
        }
    }
    // gate||up with the SwiGLU epilogue on short K: two k parts per workgroup (see kGuShortKT).
    if constexpr (MT <= 2 && !SW && GU) {
        if (KS == 1 && KW == 1 && KT <= kGuShortKT && KT % 2 == 0) {
            if (KT / 2 <= 8)
                launch_shape<MT, 1, 2 * kMfmaWaves, SW, GU, 2, 1, 8>(x, xs, M, w, s, b, y, ys, NT, KT, 1, partial, st);
            else
                launch_shape<MT, 1, 2 * kMfmaWaves, SW, GU, 2, 1, 16>(x, xs, M, w, s, b, y, ys, NT, KT, 1, partial, st);
            return;
        }
    }
    if constexpr (MT <= 2 && !SW) {
        if (range <= 8) {
            launch_shape<MT, 1, kMfmaWaves, SW, GU, 1, 1, 8>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);
            return;
        }
        if (range <= 16) {
            launch_shape<MT, 1, kMfmaWaves, SW, GU, 1, 1, 16>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);
            return;
        }
    }
    launch_shape<MT, 1, kMfmaWaves, SW, GU>(x, xs, M, w, s, b, y, ys, NT, KT, KS, partial, st);
}

template <bool SW = false>
static void launch_mfma_mt(int MT, const uint16_t* x, int64_t xs, int M, const uint8_t* w, const uint16_t* s,
                           const uint16_t* b, uint16_t* y, int64_t ys, int NT, int KT, int KS, int KW, float* partial,
                           hipStream_t st) {
    switch (MT) {
        case 1: launch_mfma<1, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
        case 2: launch_mfma<2, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
        case 3: launch_mfma<3, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
        case 4: launch_mfma<4, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
        case 6: launch_mfma<6, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
        default: launch_mfma<8, SW>(x, xs, M, w, s, b, y, ys, NT, KT, KS, KW, partial, st); break;
    }
}

static void launch_reduce(const float* partial, int KS, int M, int N, const uint16_t* b, uint16_t* y, int64_t ys,
                          hipStream_t st) {
    const dim3 grid((unsigned)ceil_div((int64_t)M * (N / 8), 256)), block(256);
    switch (KS) {
        case 2: hipLaunchKernelGGL(reduce_kernel<2>, grid, block, 0, st, partial, KS, M, N, b, y, ys); break;
        case 4: hipLaunchKernelGGL(reduce_kernel<4>, grid, block, 0, st, partial, KS, M, N, b, y, ys); break;
        case 8: hipLaunchKernelGGL(reduce_kernel<8>, grid, block, 0, st, partial, KS, M, N, b, y, ys); break;
        case 16: hipLaunchKernelGGL(reduce_kernel<16>, grid, block, 0, st, partial, KS, M, N, b, y, ys); break;
        default: hipLaunchKernelGGL(reduce_kernel<0>, grid, block, 0, st, partial, KS, M, N, b, y, ys); break;
    }
}

// ---------------------------------------------------------------------------
// Fused MLP launch (mx_w8a16_mlp_fused_partials): silu(x Wg^T) * (x Wu^T) and the split partials of
// down in one persistent launch, so that down's first weight loads overlap the end of gate||up
// instead of waiting behind a launch boundary. Workgroup i first computes gate||up group i (8 waves
// of one n-tile each: 64 activation channels, whole 128-byte lines of every row) if i < groups1,
// stores it device-coherent and counts itself in the arrival counter of each down chunk its
// channels overlap (a chunk: the k range of one k part of one split of down). It then runs down's
// workgroup (i % groups2, split i / groups2), which issues its first P stages of weights, waits for
// its chunks and reads the activations with device-coherent loads. The last workgroup to finish
// clears the counters for the next launch. Every workgroup must be resident at once (checked on the
// host from the occupancy), or a wait could stall on a workgroup that has not started; the waits
// are bounded in any case (kMlpSpinLimit). Both phases run the standalone launches' code with the
// same k order per output, so act and the partials are bit-identical to gate||up + down run apart.
// Measured on MI355X (Llama-3-8B MLP, 32 rows) it is slower than the two launches, 48-50 against
// 39.6-41.3 us: down's chunks wait for gate||up's slowest workgroups, which end 4-6 us after the
// median, and the hand-off (counter, poll, first activation loads) costs about what the launch
// boundary did. The decode step keeps the two launches unless asked (Int8DecodeModel.fuse_mlp).
constexpr int kMlpWaves = 8;
constexpr int kMlpGroupCh = kMlpWaves * kTileN / 2;  // activation channels per gate||up workgroup
constexpr int kMlpDownWn = kMlpWaves / kKParts;      // down: waves along N per k part, one n-tile each

// One 8-wave workgroup per CU at 2 or 3 waves per SIMD alike. At 2 (256 VGPRs) the kernel holds
// everything in registers; at 3 (168) gate||up streamed faster, as in its own launch (phase 1 ended
// at a median of 22 against 25 us per workgroup, the launch 45.9 against 48.5 us on MI355X at the
// Llama-3-8B MLP's 32 rows), but this build spills 20 bytes per lane there.
template <int MT>
__global__ __launch_bounds__(kMlpWaves * 64, 2) void mlp_fused_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, const uint8_t* __restrict__ wgu,
    const uint16_t* __restrict__ sgu, const uint16_t* __restrict__ bgu, uint16_t* __restrict__ act, int64_t as,
    int KT1, int NT1, const uint8_t* __restrict__ wd, const uint16_t* __restrict__ sd, int KT2, int NT2, int KS2,
    int groups2, float* __restrict__ partial, MlpWait wt) {
    constexpr int P = mfma_depth(MT);
    const int wg = blockIdx.x;
    if (wg < wt.groups) {
        gemm_body<MT, 1, kMlpWaves, P, false, true, 1, 1, 0, 1>(wg, 0, 1, x, xs, M, wgu, sgu, bgu, act, as, KT1, NT1,
                                                                nullptr, wt);
        // Every wave's stores have completed (vmcnt 0) before the workgroup counts itself.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            const int lo = wg * wt.group_ch, hi = lo + wt.group_ch - 1, chunks = KS2 * kKParts;
            for (int c = lo / wt.chunk_ch; c <= hi / wt.chunk_ch && c < chunks; ++c)
                __hip_atomic_fetch_add(wt.sync + c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    gemm_body<MT, 1, kMlpWaves, P, false, false, kKParts, 1, 0, 2>(wg % groups2, wg / groups2, KS2, act, as, M, wd, sd,
                                                                   nullptr, nullptr, 0, KT2, NT2, partial, wt);
    // Thread 0 has passed its workgroup's wait: the last one to get here clears the counters.
    if (threadIdx.x == 0) {
        const int done = __hip_atomic_fetch_add(wt.sync + kMlpDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (int)gridDim.x - 1) {
            for (int c = 0; c < KS2 * kKParts; ++c)
                __hip_atomic_store(wt.sync + c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wt.sync + kMlpDone, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

struct MlpPlan {
    int MT, KS2, groups1, groups2, grid;
};

// Workgroups of the fused kernel that fit on the current device at once, cached per device and
// instance; 0 if the runtime cannot say.
template <int MT>
static int mlp_resident() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cache[dev] == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mlp_fused_kernel<MT>, kMlpWaves * 64, 0) != hipSuccess)
            return 0;
        cache[dev] = cus * per_cu;
    }
    return cache[dev];
}

// The fused launch takes M = 5..32 rows (one or two m-tiles) where gate||up alone would run as one
// unsplit MFMA launch and down as a split one with k parts (the Llama-3-8B MLP at batch 32), and
// where all of its workgroups fit on the device at once. shape_only: skip the device check.
static bool mlp_plan(int64_t M, int64_t K, int64_t I, int64_t N, MlpPlan& mp, bool shape_only = false) {
    if (M <= kValuMaxM || M > 32 || K <= 0 || I <= 0 || N <= 0) return false;
    if (K % kTileK || I % kMlpGroupCh || N % (kTileN * kMlpDownWn)) return false;
    if (K / kTileK > (1 << 20) || 2 * I / kTileN > (1 << 24) || N / kTileN > (1 << 24) || I * 64 > 0x7fffffff)
        return false;
    const int NT1 = (int)(2 * I / kTileN), KT1 = (int)(K / kTileK);
    const int NT2 = (int)(N / kTileN), KT2 = (int)(I / kTileK);
    const Plan p1 = plan_for((int)M, NT1, KT1), p2 = plan_for((int)M, NT2, KT2);
    if (p1.valu || p1.KS != 1 || p2.valu || p2.KS < 2 || p2.KW != kKParts || p2.MT != p1.MT || p2.MT > 2) return false;
    if (KT2 % (p2.KS * kKParts) != 0 || p2.KS * kKParts > kMlpMaxChunks) return false;
    mp.MT = p2.MT;
    mp.KS2 = p2.KS;
    mp.groups1 = NT1 / kMlpWaves;
    mp.groups2 = NT2 / kMlpDownWn;
    mp.grid = mp.groups2 * mp.KS2;
    if (mp.groups1 > mp.grid || mp.grid > 65535) return false;
    if (shape_only) return true;
    return (mp.MT == 1 ? mlp_resident<1>() : mlp_resident<2>()) >= mp.grid;
}

}  // namespace w8a16
}  // namespace mx

using namespace mx;

extern "C" int mx_w8a16_quantize(const float* w, int64_t N, int64_t K, int8_t* q, uint16_t* scale, void* stream) {
    if (!w || !q || !scale) return fail(MX_ERR_NULL, "mx_w8a16_quantize: null pointer");
    if (N <= 0 || K <= 0) return fail(MX_ERR_INVALID, "mx_w8a16_quantize: N and K must be positive (N=%lld K=%lld)",
                                      (long long)N, (long long)K);
    if (N > 0x7fffffff) return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_quantize: N too large");
    hipLaunchKernelGGL(w8a16::quantize_kernel, dim3((unsigned)N), dim3(256), 0, as_stream(stream), w, K, q, scale);
    return check_launch("mx_w8a16_quantize");
}

extern "C" int mx_w8a16_pack(const int8_t* q, int64_t N, int64_t K, uint8_t* packed, void* stream) {
    if (!q || !packed) return fail(MX_ERR_NULL, "mx_w8a16_pack: null pointer");
    if (N <= 0 || K <= 0 || N % w8a16::kTileN || K % w8a16::kTileK)
        return fail(MX_ERR_INVALID, "mx_w8a16_pack: need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)",
                    (long long)N, (long long)K);
    if (!aligned(q, 16) || !aligned(packed, 16)) return fail(MX_ERR_ALIGNMENT, "mx_w8a16_pack: 16-byte alignment");
    const int64_t slots = N * K / 16;
    const int64_t blocks = ceil_div(slots, 256);
    if (blocks > 0x7fffffff) return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_pack: matrix too large");
    hipLaunchKernelGGL(w8a16::pack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), q, K,
                       K / w8a16::kTileK, slots, packed);
    return check_launch("mx_w8a16_pack");
}

extern "C" size_t mx_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || N % w8a16::kTileN || K % w8a16::kTileK) return 0;
    const int mc = (int)(M < w8a16::kMaxRows ? M : w8a16::kMaxRows);  // rows are processed in chunks
    return w8a16::workspace_for(mc, (int)(N / w8a16::kTileN), (int)(K / w8a16::kTileK));
}

extern "C" int mx_w8a16_linear(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                               const uint16_t* scale, const uint16_t* bias, uint16_t* y, int64_t N, int64_t y_stride,
                               void* workspace, size_t workspace_bytes, void* stream) {
    if (!x || !packed || !scale || !y) return fail(MX_ERR_NULL, "mx_w8a16_linear: null pointer");
    if (M < 0 || N <= 0 || K <= 0) return fail(MX_ERR_INVALID, "mx_w8a16_linear: bad sizes M=%lld N=%lld K=%lld",
                                               (long long)M, (long long)N, (long long)K);
    if (N % w8a16::kTileN || K % w8a16::kTileK)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear: need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)",
                    (long long)N, (long long)K);
    if (x_stride < K || y_stride < N)
        return fail(MX_ERR_INVALID, "mx_w8a16_linear: row strides must cover K and N");
    if (!aligned(x, 16) || (x_stride % 8) != 0 || !aligned(packed, 16))
        return fail(MX_ERR_ALIGNMENT, "mx_w8a16_linear: x rows and packed weights must be 16-byte aligned");
    if (N / w8a16::kTileN > 0x7fffffff || K / w8a16::kTileK > 0x7fffffff || K * 64 > 0x7fffffff)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear: matrix too large");
    if (workspace && !aligned(workspace, 16))
        return fail(MX_ERR_ALIGNMENT, "mx_w8a16_linear: workspace must be 16-byte aligned");
    if (M == 0) return MX_OK;
    const int NT = (int)(N / w8a16::kTileN);
    const int KT = (int)(K / w8a16::kTileK);
    hipStream_t st = as_stream(stream);
    float* partial = static_cast<float*>(workspace);
    for (int64_t m0 = 0; m0 < M; m0 += w8a16::kMaxRows) {
        const int mc = (int)((M - m0) < w8a16::kMaxRows ? (M - m0) : w8a16::kMaxRows);
        const uint16_t* xc = x + m0 * x_stride;
        uint16_t* yc = y + m0 * y_stride;
        w8a16::Plan pl = w8a16::plan_for(mc, NT, KT);
        // Split-K needs the caller's workspace; without enough of it run unsplit.
        if (pl.KS > 1 && (!workspace || workspace_bytes < w8a16::workspace_for(mc, NT, KT))) pl.KS = pl.KW = 1;
        if (pl.valu) {
            w8a16::launch_gemv_m(mc, xc, x_stride, packed, scale, bias, yc, y_stride, NT, KT, st);
        } else {
            w8a16::launch_mfma_mt(pl.MT, xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, pl.KS, pl.KW, partial,
                                  st);
            if (pl.KS > 1) w8a16::launch_reduce(partial, pl.KS, mc, (int)N, bias, yc, y_stride, st);
        }
        const int rc = check_launch("mx_w8a16_linear");
        if (rc != MX_OK) return rc;
    }
    return MX_OK;
}

extern "C" int mx_w8a16_splits(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || M > w8a16::kMaxRows || N <= 0 || K <= 0 || N % w8a16::kTileN || K % w8a16::kTileK) return 1;
    return w8a16::plan_for((int)M, (int)(N / w8a16::kTileN), (int)(K / w8a16::kTileK)).KS;
}

extern "C" int mx_w8a16_linear_partials(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride,
                                        const uint8_t* packed, const uint16_t* scale, int64_t N, float* partials,
                                        size_t partials_bytes, void* stream) {
    if (!x || !packed || !scale || !partials) return fail(MX_ERR_NULL, "mx_w8a16_linear_partials: null pointer");
    if (M <= 0 || M > w8a16::kMaxRows || N <= 0 || K <= 0)
        return fail(MX_ERR_INVALID, "mx_w8a16_linear_partials: need 1 <= M <= %d and positive N, K", w8a16::kMaxRows);
    if (N % w8a16::kTileN || K % w8a16::kTileK)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear_partials: need N %% 16 == 0 and K %% 64 == 0");
    if (x_stride < K) return fail(MX_ERR_INVALID, "mx_w8a16_linear_partials: x row stride must cover K");
    if (!aligned(x, 16) || (x_stride % 8) != 0 || !aligned(packed, 16) || !aligned(partials, 16))
        return fail(MX_ERR_ALIGNMENT, "mx_w8a16_linear_partials: x rows, weights and partials must be 16-byte aligned");
    if (N / w8a16::kTileN > 0x7fffffff || K * 64 > 0x7fffffff)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear_partials: matrix too large");
    const int NT = (int)(N / w8a16::kTileN);
    const int KT = (int)(K / w8a16::kTileK);
    const w8a16::Plan pl = w8a16::plan_for((int)M, NT, KT);
    if (pl.valu || pl.KS == 1)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear_partials: shape is not split (mx_w8a16_splits == 1); "
                                        "use mx_w8a16_linear");
    if (partials_bytes < (size_t)pl.KS * M * N * sizeof(float))
        return fail(MX_ERR_WORKSPACE, "mx_w8a16_linear_partials: partials need %zu bytes, got %zu",
                    (size_t)pl.KS * M * N * sizeof(float), partials_bytes);
    w8a16::launch_mfma_mt(pl.MT, x, x_stride, (int)M, packed, scale, nullptr, nullptr, 0, NT, KT, pl.KS, pl.KW, partials,
                          as_stream(stream));
    return check_launch("mx_w8a16_linear_partials");
}

// SwiGLU-input variants: x = silu(gate_up[:, :K]) * gate_up[:, K:2K], formed in the x
// staging of the MFMA kernel (M >= 5).
static int swiglu_checks(const char* what, const uint16_t* gu, int64_t M, int64_t K, int64_t gu_stride,
                         const uint8_t* packed, const uint16_t* scale, int64_t N) {
    if (!gu || !packed || !scale) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (M <= w8a16::kValuMaxM || M > w8a16::kMaxRows || N <= 0 || K <= 0)
        return fail(MX_ERR_UNSUPPORTED, "%s: needs %d < M <= 128 and positive N, K (M=%lld)", what, w8a16::kValuMaxM,
                    (long long)M);
    if (N % w8a16::kTileN || K % w8a16::kTileK)
        return fail(MX_ERR_UNSUPPORTED, "%s: need N %% 16 == 0 and K %% 64 == 0", what);
    if (gu_stride < 2 * K) return fail(MX_ERR_INVALID, "%s: gate_up row stride must cover 2K", what);
    if (!aligned(gu, 16) || (gu_stride % 8) != 0 || !aligned(packed, 16))
        return fail(MX_ERR_ALIGNMENT, "%s: gate_up rows and weights must be 16-byte aligned", what);
    if (N / w8a16::kTileN > 0x7fffffff || K * 64 > 0x7fffffff) return fail(MX_ERR_UNSUPPORTED, "%s: too large", what);
    return MX_OK;
}

extern "C" int mx_w8a16_linear_swiglu(const uint16_t* gate_up, int64_t M, int64_t K, int64_t gu_stride,
                                      const uint8_t* packed, const uint16_t* scale, const uint16_t* bias, uint16_t* y,
                                      int64_t N, int64_t y_stride, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    int rc = swiglu_checks("mx_w8a16_linear_swiglu", gate_up, M, K, gu_stride, packed, scale, N);
    if (rc != MX_OK) return rc;
    if (!y) return fail(MX_ERR_NULL, "mx_w8a16_linear_swiglu: null output");
    if (y_stride < N) return fail(MX_ERR_INVALID, "mx_w8a16_linear_swiglu: y row stride must cover N");
    if (workspace && !aligned(workspace, 16))
        return fail(MX_ERR_ALIGNMENT, "mx_w8a16_linear_swiglu: workspace must be 16-byte aligned");
    const int NT = (int)(N / w8a16::kTileN), KT = (int)(K / w8a16::kTileK);
    w8a16::Plan pl = w8a16::plan_for((int)M, NT, KT);
    if (pl.KS > 1 && (!workspace || workspace_bytes < w8a16::workspace_for((int)M, NT, KT))) pl.KS = pl.KW = 1;
    float* partial = static_cast<float*>(workspace);
    hipStream_t st = as_stream(stream);
    w8a16::launch_mfma_mt<true>(pl.MT, gate_up, gu_stride, (int)M, packed, scale, bias, y, y_stride, NT, KT, pl.KS, pl.KW,
                                partial, st);
    if (pl.KS > 1) w8a16::launch_reduce(partial, pl.KS, (int)M, (int)N, bias, y, y_stride, st);
    return check_launch("mx_w8a16_linear_swiglu");
}

extern "C" int mx_w8a16_linear_partials_swiglu(const uint16_t* gate_up, int64_t M, int64_t K, int64_t gu_stride,
                                               const uint8_t* packed, const uint16_t* scale, int64_t N,
                                               float* partials, size_t partials_bytes, void* stream) {
    int rc = swiglu_checks("mx_w8a16_linear_partials_swiglu", gate_up, M, K, gu_stride, packed, scale, N);
    if (rc != MX_OK) return rc;
    if (!partials) return fail(MX_ERR_NULL, "mx_w8a16_linear_partials_swiglu: null partials");
    if (!aligned(partials, 16)) return fail(MX_ERR_ALIGNMENT, "mx_w8a16_linear_partials_swiglu: partials alignment");
    const int NT = (int)(N / w8a16::kTileN), KT = (int)(K / w8a16::kTileK);
    const w8a16::Plan pl = w8a16::plan_for((int)M, NT, KT);
    if (pl.KS == 1) return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_linear_partials_swiglu: shape is not split");
    if (partials_bytes < (size_t)pl.KS * M * N * sizeof(float))
        return fail(MX_ERR_WORKSPACE, "mx_w8a16_linear_partials_swiglu: partials need %zu bytes",
                    (size_t)pl.KS * M * N * sizeof(float));
    w8a16::launch_mfma_mt<true>(pl.MT, gate_up, gu_stride, (int)M, packed, scale, nullptr, nullptr, 0, NT, KT, pl.KS, pl.KW,
                                partials, as_stream(stream));
    return check_launch("mx_w8a16_linear_partials_swiglu");
}

extern "C" int mx_w8a16_gateup_swiglu(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride, const uint8_t* packed,
                                      const uint16_t* scale, const uint16_t* bias, uint16_t* y, int64_t I,
                                      int64_t y_stride, void* stream) {
    if (!x || !packed || !scale || !y) return fail(MX_ERR_NULL, "mx_w8a16_gateup_swiglu: null pointer");
    if (M <= 0 || M > 0x7fffffff || I <= 0 || K <= 0)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_gateup_swiglu: needs M >= 1 (M=%lld)", (long long)M);
    if (I % 8 || K % w8a16::kTileK)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_gateup_swiglu: need I %% 8 == 0 and K %% 64 == 0");
    if (x_stride < K || y_stride < I) return fail(MX_ERR_INVALID, "mx_w8a16_gateup_swiglu: row strides too short");
    if (!aligned(x, 16) || (x_stride % 8) != 0 || !aligned(packed, 16))
        return fail(MX_ERR_ALIGNMENT, "mx_w8a16_gateup_swiglu: x rows and weights must be 16-byte aligned");
    const int NT = (int)(2 * I / w8a16::kTileN), KT = (int)(K / w8a16::kTileK);
    if ((int64_t)NT * w8a16::kTileN != 2 * I || K * 64 > 0x7fffffff)
        return fail(MX_ERR_UNSUPPORTED, "mx_w8a16_gateup_swiglu: bad shape");
    // Rows in chunks of at most kMaxRows, as mx_w8a16_linear: the VALU GEMV where that entry
    // would take it (M <= 4 on shapes that split), else one unsplit MFMA launch, also where
    // mx_w8a16_linear would split K: the epilogue needs the whole sum, and on such (small)
    // shapes one launch without K split costs less than a split launch plus a SwiGLU launch
    // (the Qwen2-0.5B MLP at batch 16).
    hipStream_t st = as_stream(stream);
    for (int64_t m0 = 0; m0 < M; m0 += w8a16::kMaxRows) {
        const int mc = (int)(M - m0 < w8a16::kMaxRows ? M - m0 : w8a16::kMaxRows);
        const uint16_t* xc = x + m0 * x_stride;
        uint16_t* yc = y + m0 * y_stride;
        const w8a16::Plan pl = w8a16::plan_for(mc, NT, KT);
        if (pl.valu) {
            w8a16::launch_gemv_m<true>(mc, xc, x_stride, packed, scale, bias, yc, y_stride, NT, KT, st);
            continue;
        }
        switch (pl.MT) {
            case 1: w8a16::launch_mfma<1, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
            case 2: w8a16::launch_mfma<2, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
            case 3: w8a16::launch_mfma<3, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
            case 4: w8a16::launch_mfma<4, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
            case 6: w8a16::launch_mfma<6, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
            default: w8a16::launch_mfma<8, false, true>(xc, x_stride, mc, packed, scale, bias, yc, y_stride, NT, KT, 1, 1, nullptr, st); break;
        }
    }
    return check_launch("mx_w8a16_gateup_swiglu");
}

extern "C" int mx_w8a16_mlp_fused_supported(int64_t M, int64_t K, int64_t I, int64_t N) {
    w8a16::MlpPlan mp{};
    return w8a16::mlp_plan(M, K, I, N, mp) ? 1 : 0;
}

extern "C" int mx_w8a16_mlp_fused_partials(const uint16_t* x, int64_t M, int64_t K, int64_t x_stride,
                                           const uint8_t* gu_packed, const uint16_t* gu_scale,
                                           const uint16_t* gu_bias, int64_t I, uint16_t* act, int64_t act_stride,
                                           const uint8_t* down_packed, const uint16_t* down_scale, int64_t N,
                                           float* partials, size_t partials_bytes, int32_t* sync, void* stream) {
    const char* what = "mx_w8a16_mlp_fused_partials";
    if (!x || !gu_packed || !gu_scale || !act || !down_packed || !down_scale || !partials || !sync)
        return fail(MX_ERR_NULL, "%s: null pointer", what);
    w8a16::MlpPlan mp{};
    if (!w8a16::mlp_plan(M, K, I, N, mp, true))
        return fail(MX_ERR_UNSUPPORTED, "%s: shape M=%lld K=%lld I=%lld N=%lld does not take the fused launch", what,
                    (long long)M, (long long)K, (long long)I, (long long)N);
    if (!w8a16::mlp_plan(M, K, I, N, mp))
        return fail(MX_ERR_UNSUPPORTED, "%s: the %d workgroups of the fused launch do not fit on this device at once",
                    what, mp.grid);
    if (x_stride < K || act_stride < I) return fail(MX_ERR_INVALID, "%s: row strides must cover K and I", what);
    if (!aligned(x, 16) || (x_stride % 8) != 0 || !aligned(gu_packed, 16) || !aligned(down_packed, 16) ||
        !aligned(partials, 16) || !aligned(sync, 4))
        return fail(MX_ERR_ALIGNMENT, "%s: x rows, weights and partials must be 16-byte aligned", what);
    // Each gate||up workgroup writes whole 128-byte lines of every activation row, so that no line is
    // written from two XCDs.
    if (!aligned(act, 128) || (act_stride * 2) % 128 != 0)
        return fail(MX_ERR_ALIGNMENT, "%s: act must be 128-byte aligned with a row stride of a multiple of 64", what);
    if (partials_bytes < (size_t)mp.KS2 * M * N * sizeof(float))
        return fail(MX_ERR_WORKSPACE, "%s: partials need %zu bytes, got %zu", what,
                    (size_t)mp.KS2 * M * N * sizeof(float), partials_bytes);
    w8a16::MlpWait wt;
    wt.sync = sync;
    wt.chunk_ch = (int)(I / (mp.KS2 * w8a16::kKParts));
    wt.group_ch = w8a16::kMlpGroupCh;
    wt.groups = mp.groups1;
    const int NT1 = (int)(2 * I / w8a16::kTileN), KT1 = (int)(K / w8a16::kTileK);
    const int NT2 = (int)(N / w8a16::kTileN), KT2 = (int)(I / w8a16::kTileK);
    hipStream_t st = as_stream(stream);
    if (mp.MT == 1)
        hipLaunchKernelGGL(w8a16::mlp_fused_kernel<1>, dim3(mp.grid), dim3(w8a16::kMlpWaves * 64), 0, st, x, x_stride,
                           (int)M, gu_packed, gu_scale, gu_bias, act, act_stride, KT1, NT1, down_packed, down_scale, KT2,
                           NT2, mp.KS2, mp.groups2, partials, wt);
    else
        hipLaunchKernelGGL(w8a16::mlp_fused_kernel<2>, dim3(mp.grid), dim3(w8a16::kMlpWaves * 64), 0, st, x, x_stride,
                           (int)M, gu_packed, gu_scale, gu_bias, act, act_stride, KT1, NT1, down_packed, down_scale, KT2,
                           NT2, mp.KS2, mp.groups2, partials, wt);
    return check_launch(what);
}
