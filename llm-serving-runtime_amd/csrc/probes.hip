// Calibration probes of libmxdecode (no reference counterpart; used by bench.py --workload probes).
//
// They measure what the design of the decode kernels leans on, on the GPU at hand:
//   * mx_stream_probe: how fast G workgroups of T threads stream contiguous runs of B bytes each
//     (what one CU can stream, and how many CUs and bytes a launch needs to reach the chip's rate);
//   * mx_launch_probe: what a launch costs inside a HIP graph when it does nothing, or writes a
//     given number of bytes (the floor under every small kernel of the decode step).
// Neither writes anything it was not asked to: the stream probe folds the data it reads into an xor
// that is stored only when it equals a magic value (never, in practice), so the loads stay.
#include "common.h"

namespace mx {
namespace probe {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Workgroup w reads bytes [w * per_wg, (w + 1) * per_wg) of src with non-temporal 16-byte loads,
// U loads in flight per thread (consecutive threads read consecutive 16-byte chunks).
template <int T, int U>
__global__ __launch_bounds__(T) void stream_kernel(const u32x4v* __restrict__ src, int64_t chunks_per_wg,
                                                   int32_t* __restrict__ sink) {
    const u32x4v* p = src + (int64_t)blockIdx.x * chunks_per_wg;
    uint32_t acc = 0;
    for (int64_t i0 = threadIdx.x; i0 < chunks_per_wg; i0 += (int64_t)T * U) {
        u32x4v v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * T;
            v[u] = __builtin_nontemporal_load(p + (i < chunks_per_wg ? i : chunks_per_wg - 1));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = (int32_t)acc;
}

// Empty: nothing but the launch.
__global__ __launch_bounds__(256) void empty_kernel() {}

// Workgroup w writes its chunks_per_wg 16-byte chunks of dst (thread-strided, coalesced).
__global__ __launch_bounds__(256) void write_kernel(uint4* __restrict__ dst, int64_t chunks_per_wg) {
    uint4* p = dst + (int64_t)blockIdx.x * chunks_per_wg;
    const uint32_t v = blockIdx.x;
    for (int64_t i = threadIdx.x; i < chunks_per_wg; i += 256) p[i] = uint4{v, v, v, v};
}

// Wave w of `waves` reads the runs [w * n / waves, (w + 1) * n / waves) of a list of byte offsets
// into base, each run RUN16 16-byte chunks read as RUN16 / 64 coalesced 1 KiB loads (lane l reads
// chunks l, l + 64, ...), R runs in flight per wave; STREAM selects non-temporal loads. The gather
// pattern of paged attention without its math: which runs, how many in flight, what policy.
// An offset outside [0, base_bytes - run bytes] reads run 0 instead, and offsets are rounded down to
// 16 bytes, so no offset list makes the probe read outside the buffer.
// PATTERN 0: 1 KiB contiguous per load instruction. PATTERN 1 and 2 (8 KiB runs: a 16-token K tile of
// head_dim 128 followed by its V tile, the interleaved pool): the paged-attention kernel's operand
// loads, K as 4 instructions of 16 token rows x 64 bytes (lane (r, g) = (l % 16, l / 16) reads row r,
// bytes 64 kk + 16 g) and V as 4 instructions of 4 token rows x 256 bytes (row 4 g + jj, bytes 16 r);
// 1 streams every load, 2 loads the first half of each K line with the default policy, as the kernel.
// PATTERN 3: K through LDS, V as in 1: 4 streaming global->LDS loads per K tile, each 4 whole token rows
// (1 KiB, lane l of load i carries row 4 i + l / 16, 16-byte chunk (l % 16) ^ (row % 16)), then the
// operand layout of 1 read back from LDS (the xor makes the 16 rows of a read hit distinct banks).
// PATTERN 4: K as in 3, with operand row r holding token 4 (r % 4) + r / 4, so that the tokens a V load
// needs (4 jj + g for lane group g) are 4 consecutive rows: each V load reads 1 KiB contiguous.
template <int RUN16, int R, bool STREAM, int PATTERN = 0>
__global__ __launch_bounds__(256) void run_gather_kernel(const u32x4v* __restrict__ base, int64_t base_bytes,
                                                         const int64_t* __restrict__ offsets, int64_t n_runs,
                                                         int waves, int32_t* __restrict__ sink) {
    static_assert(PATTERN == 0 || RUN16 == 512, "operand patterns: 8 KiB runs");
    constexpr int L = RUN16 / 64;  // load instructions per run
    const int wave = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    // PATTERN 3, 4: each wave's K tiles (R of 256 16-byte chunks); unused by the other patterns.
    __shared__ u32x4v k_lds[PATTERN >= 3 ? 4 * R * 256 : 1];
    if (wave >= waves) return;
    const int64_t lo = n_runs * wave / waves, hi = n_runs * (wave + 1) / waves;
    uint32_t acc = 0;
    for (int64_t r0 = lo; r0 < hi; r0 += R) {
        u32x4v v[R][L];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t ri = r0 + r < hi ? r0 + r : hi - 1;
            int64_t off = offsets[ri];
            if ((uint64_t)off > (uint64_t)(base_bytes - RUN16 * 16)) off = 0;
            if constexpr (PATTERN == 0) {
                const u32x4v* p = base + (off >> 4) + lane;
#pragma unroll
                for (int j = 0; j < L; ++j) {
                    if constexpr (STREAM) v[r][j] = __builtin_nontemporal_load(p + 64 * j);
                    else v[r][j] = p[64 * j];
                }
            } else if constexpr (PATTERN >= 3) {
                u32x4v* kw = k_lds + ((threadIdx.x >> 6) * R + r) * 256;
                const int row_in = lane >> 4, ch = lane & 15;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 4 * i + row_in;
                    __builtin_amdgcn_global_load_lds(static_cast<const void*>(base + (off >> 4) + row * 16 + (ch ^ row)),
                                                     (__attribute__((address_space(3))) void*)(kw + 64 * i),
                                                     16, 0, 2);
                }
                const int rr = lane & 15, g = lane >> 4;
                // V row 4 g + jj (3) or 4 jj + g (4), chunk rr
                const u32x4v* vv = base + (off >> 4) + 256 + (PATTERN == 3 ? g * 64 : g * 16) + rr;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) v[r][4 + jj] = __builtin_nontemporal_load(vv + (PATTERN == 3 ? 16 : 64) * jj);
            } else {
                const int rr = lane & 15, g = lane >> 4;
                const u32x4v* k = base + (off >> 4) + rr * 16 + g;         // row rr, 16-byte chunk g
                const u32x4v* vv = base + (off >> 4) + 256 + g * 64 + rr;  // V tile: row 4 g, chunk rr
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    if (PATTERN == 2 && (kk & 1) == 0) v[r][kk] = k[4 * kk];
                    else v[r][kk] = __builtin_nontemporal_load(k + 4 * kk);
                }
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) v[r][4 + jj] = __builtin_nontemporal_load(vv + 16 * jj);
            }
        }
        if constexpr (PATTERN >= 3) {
            // The global->LDS loads are not tracked by the compiler's waits: wait for every load of
            // the round (vmcnt(0)) before reading K back; the reads of a round finish (their values
            // are consumed below) before the next round's loads overwrite the buffers.
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __builtin_amdgcn_sched_barrier(0);
            const int rr = lane & 15, g = lane >> 4;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const u32x4v* kw = k_lds + ((threadIdx.x >> 6) * R + r) * 256;
                const int t = PATTERN == 3 ? rr : 4 * (rr & 3) + (rr >> 2);  // the token of operand row rr
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) v[r][kk] = kw[64 * (t >> 2) + 16 * (t & 3) + ((g + 4 * kk) ^ t)];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < L; ++j) acc ^= v[r][j].x ^ v[r][j].y ^ v[r][j].z ^ v[r][j].w;
        if constexpr (PATTERN >= 3) __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x9e3779b9u) sink[0] = (int32_t)acc;
}

}  // namespace probe
}  // namespace mx

using namespace mx;

extern "C" int mx_stream_probe(const void* src, int64_t src_bytes, int64_t offset, int64_t bytes_per_wg,
                               int32_t workgroups, int32_t threads, int32_t* sink, void* stream) {
    const char* what = "mx_stream_probe";
    clear_error();
    if (!src || !sink) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (workgroups <= 0 || bytes_per_wg <= 0 || bytes_per_wg % 16 || offset < 0 || offset % 16)
        return fail(MX_ERR_INVALID, "%s: need workgroups > 0 and 16-byte multiples for bytes_per_wg and offset", what);
    if (offset + (int64_t)workgroups * bytes_per_wg > src_bytes)
        return fail(MX_ERR_INVALID, "%s: %d x %lld bytes from offset %lld exceed the %lld-byte buffer", what,
                    workgroups, (long long)bytes_per_wg, (long long)offset, (long long)src_bytes);
    if (!aligned(src, 16)) return fail(MX_ERR_ALIGNMENT, "%s: src must be 16-byte aligned", what);
    const auto* p = reinterpret_cast<const probe::u32x4v*>(static_cast<const char*>(src) + offset);
    const int64_t chunks = bytes_per_wg / 16;
    hipStream_t st = as_stream(stream);
    switch (threads) {
        case 256: hipLaunchKernelGGL((probe::stream_kernel<256, 4>), dim3(workgroups), dim3(256), 0, st, p, chunks, sink); break;
        case 512: hipLaunchKernelGGL((probe::stream_kernel<512, 4>), dim3(workgroups), dim3(512), 0, st, p, chunks, sink); break;
        case 1024: hipLaunchKernelGGL((probe::stream_kernel<1024, 4>), dim3(workgroups), dim3(1024), 0, st, p, chunks, sink); break;
        default: return fail(MX_ERR_UNSUPPORTED, "%s: threads must be 256, 512 or 1024", what);
    }
    return check_launch(what);
}

extern "C" int mx_launch_probe(void* dst, int64_t dst_bytes, int64_t bytes, int32_t workgroups, void* stream) {
    const char* what = "mx_launch_probe";
    clear_error();
    if (workgroups <= 0 || bytes < 0 || bytes % (16 * (int64_t)workgroups))
        return fail(MX_ERR_INVALID, "%s: bytes must be a multiple of 16 x workgroups", what);
    hipStream_t st = as_stream(stream);
    if (bytes == 0) {
        hipLaunchKernelGGL(probe::empty_kernel, dim3(workgroups), dim3(256), 0, st);
    } else {
        if (!dst) return fail(MX_ERR_NULL, "%s: null dst", what);
        if (bytes > dst_bytes) return fail(MX_ERR_INVALID, "%s: %lld bytes exceed the %lld-byte buffer", what,
                                            (long long)bytes, (long long)dst_bytes);
        if (!aligned(dst, 16)) return fail(MX_ERR_ALIGNMENT, "%s: dst must be 16-byte aligned", what);
        hipLaunchKernelGGL(probe::write_kernel, dim3(workgroups), dim3(256), 0, st, static_cast<uint4*>(dst),
                           bytes / 16 / workgroups);
    }
    return check_launch(what);
}

extern "C" int mx_run_gather_probe(const void* base, int64_t base_bytes, const int64_t* offsets, int64_t n_runs,
                                   int32_t run_bytes, int32_t waves, int32_t in_flight, int32_t streaming,
                                   int32_t pattern, int32_t* sink, void* stream) {
    const char* what = "mx_run_gather_probe";
    clear_error();
    if (!base || !offsets || !sink) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (n_runs <= 0 || waves <= 0 || base_bytes < run_bytes)
        return fail(MX_ERR_INVALID, "%s: need runs, waves > 0 and a buffer of at least one run", what);
    if (run_bytes != 4096 && run_bytes != 8192) return fail(MX_ERR_UNSUPPORTED, "%s: run_bytes 4096 or 8192", what);
    if (!aligned(base, 16)) return fail(MX_ERR_ALIGNMENT, "%s: base must be 16-byte aligned", what);
    hipStream_t st = as_stream(stream);
    const auto* b = static_cast<const probe::u32x4v*>(base);
    const dim3 grid((unsigned)ceil_div(waves, 4)), block(256);
    if (pattern >= 1 && pattern <= 4) {
        if (run_bytes != 8192) return fail(MX_ERR_UNSUPPORTED, "%s: the operand patterns take 8192-byte runs", what);
        if (in_flight != 2) return fail(MX_ERR_UNSUPPORTED, "%s: the operand patterns take 2 runs in flight", what);
        if (pattern == 1)
            hipLaunchKernelGGL((probe::run_gather_kernel<512, 2, true, 1>), grid, block, 0, st, b, base_bytes, offsets,
                               n_runs, waves, sink);
        else if (pattern == 3)
            hipLaunchKernelGGL((probe::run_gather_kernel<512, 2, true, 3>), grid, block, 0, st, b, base_bytes, offsets,
                               n_runs, waves, sink);
        else if (pattern == 4)
            hipLaunchKernelGGL((probe::run_gather_kernel<512, 2, true, 4>), grid, block, 0, st, b, base_bytes, offsets,
                               n_runs, waves, sink);
        else
            hipLaunchKernelGGL((probe::run_gather_kernel<512, 2, true, 2>), grid, block, 0, st, b, base_bytes, offsets,
                               n_runs, waves, sink);
        return check_launch(what);
    }
    if (pattern != 0) return fail(MX_ERR_INVALID, "%s: pattern must be 0 to 4", what);
#define MX_RG(RB, R, S)                                                                                          \
    if (run_bytes == RB && in_flight == R && (streaming != 0) == S) {                                           \
        hipLaunchKernelGGL((probe::run_gather_kernel<RB / 16, R, S>), grid, block, 0, st, b, base_bytes, offsets,  \
                           n_runs, waves, sink);                                                                \
        return check_launch(what);                                                                              \
    }
    MX_RG(8192, 1, true) MX_RG(8192, 2, true) MX_RG(8192, 3, true) MX_RG(8192, 4, true) MX_RG(8192, 6, true)
    MX_RG(8192, 1, false) MX_RG(8192, 2, false) MX_RG(8192, 3, false) MX_RG(8192, 4, false) MX_RG(8192, 6, false)
    MX_RG(4096, 2, true) MX_RG(4096, 4, true) MX_RG(4096, 2, false) MX_RG(4096, 4, false)
#undef MX_RG
    return fail(MX_ERR_UNSUPPORTED, "%s: in_flight %d not built for %d-byte runs (8192: 1, 2, 3, 4, 6; 4096: 2, 4)",
                what, in_flight, run_bytes);
}
