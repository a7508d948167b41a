// Calibration probes of libmxdecode (no reference counterpart; used by bench.py --workload probes).
//
// They measure what the design of the decode kernels leans on, on the GPU at hand:
//   * mx_stream_probe: how fast G workgroups of T threads stream contiguous runs of B bytes each
//     (what one CU can stream, and how many CUs and bytes a launch needs to reach the chip's rate);
//   * mx_launch_probe: what a launch costs inside a HIP graph when it does nothing, or writes a
//     given number of bytes (the floor under every small kernel of the decode step);
//   * mx_run_gather_probe: the K/V gather of paged attention without its math;
//   * mx_handoff_probe, mx_barrier_probe, mx_chain_probe: what handing data between the workgroups
//     of one launch costs (last-arriver sums, grid barriers, a persistent chain of phases) against
//     a launch boundary: the measurements behind keeping the decode step a graph of kernels.
// None writes anything it was not asked to: the reading probes fold the data they read into an xor
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

// ---------------------------------------------------------------------------
// Hand-offs between the workgroups of one launch (mx_handoff_probe, mx_barrier_probe,
// mx_chain_probe): what a fused or persistent kernel would pay instead of a launch boundary.
// Device-coherent accesses are agent-scope relaxed atomics: their stores write through the XCD's
// L2 and their loads read past it, so a workgroup on another XCD sees them without fences. Waits
// are bounded (kSpinLimit polls, then err bit 1 and no further waits by that thread), and the
// launches that wait check on the host that every workgroup is resident at once.
// ---------------------------------------------------------------------------
constexpr int kSpinLimit = 1 << 16;
constexpr int kCounters = 8;   // sync words 0-7: arrival counters (workgroup w counts in w % 8)
constexpr int kDoneWord = 8;   // sync word 8: workgroups finished (the last one clears the words)
constexpr int kFlagWords = 16; // sync words 16..16+N: one flag per workgroup (barrier mode 1)

__device__ __forceinline__ void store_coherent(int32_t* p, uint4 v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p) + 1, (uint64_t)v.z | ((uint64_t)v.w << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 load_coherent(int32_t* p) {
    const uint64_t a = __hip_atomic_load(reinterpret_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(reinterpret_cast<uint64_t*>(p) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return uint4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// Polls *c until it reaches want; false after kSpinLimit polls.
__device__ __forceinline__ bool poll_at_least(int32_t* c, int want) {
    for (int polls = 0; __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < want; ++polls) {
        if (polls >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

// Workgroups w < N with w % kCounters == c.
__device__ __forceinline__ int counter_members(int c, int N) { return (N - c + kCounters - 1) / kCounters; }

// Thread 0 counts its workgroup as finished; the last workgroup clears the counters, the done word
// and `flags` flag words for the next launch (every workgroup has passed its last wait by then).
__device__ __forceinline__ void finish_and_clear(int32_t* sync, int flags) {
    if (threadIdx.x != 0) return;
    if (__hip_atomic_fetch_add(sync + kDoneWord, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != (int)gridDim.x - 1)
        return;
    for (int c = 0; c < kCounters; ++c) __hip_atomic_store(sync + c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int f = 0; f < flags; ++f)
        __hip_atomic_store(sync + kFlagWords + f, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(sync + kDoneWord, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Hand-off probe: workgroup w (256 threads) writes an 8 KiB fp32 partial, value (31 w + i) & 1023 at
// float i; the G partials of group w / G are summed in index order into out[group]. MODE:
//   0: the partials only; 1: the partials, then handoff_reduce_kernel (one workgroup per group);
//   2: the group's last workgroup to take a ticket sums them: every thread releases its stores with
//      an agent-scope release fence before the ticket, the last arriver acquires with an agent-scope
//      acquire fence and reads plain;
//   3: as 2 with sequentially consistent agent-scope fences (__threadfence) in both places;
//   4: as 2 without fences: device-coherent partial stores and loads, each wave waiting for its
//      stores before the ticket.
// The last arriver clears its group's ticket for the next launch.
constexpr int kHandoffThreads = 256, kHandoffFloats = 2048;

__device__ __forceinline__ float handoff_value(int wg, int i) { return (float)((wg * 31 + i) & 1023); }

// Thread t sums floats 4t .. 4t + 3 and 1024 + 4t .. 1024 + 4t + 3 of the G partials at p.
template <bool COHERENT>
__device__ __forceinline__ void sum_partials(float* p, float* __restrict__ o, int G) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = h * 1024 + (int)threadIdx.x * 4;
        float4 s = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int j = 0; j < G; ++j) {
            float* q = p + (int64_t)j * kHandoffFloats + i;
            float4 v;
            if constexpr (COHERENT) {
                const uint4 u = load_coherent(reinterpret_cast<int32_t*>(q));
                v = float4{__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
            } else {
                v = *reinterpret_cast<const float4*>(q);
            }
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        *reinterpret_cast<float4*>(o + i) = s;
    }
}

template <int MODE>
__global__ __launch_bounds__(kHandoffThreads) void handoff_kernel(float* part, float* __restrict__ out,
                                                                 int32_t* __restrict__ tickets, int G) {
    __shared__ int last;
    const int wg = blockIdx.x, grp = wg / G;
    float* mine = part + (int64_t)wg * kHandoffFloats;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = h * 1024 + (int)threadIdx.x * 4;
        const float4 v = {handoff_value(wg, i), handoff_value(wg, i + 1), handoff_value(wg, i + 2),
                          handoff_value(wg, i + 3)};
        if constexpr (MODE == 4)
            store_coherent(reinterpret_cast<int32_t*>(mine + i),
                           uint4{__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)});
        else
            *reinterpret_cast<float4*>(mine + i) = v;
    }
    if constexpr (MODE >= 2) {
        if constexpr (MODE == 2) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        else if constexpr (MODE == 3) __threadfence();
        else __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(tickets + grp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1;
        __syncthreads();
        if (!last) return;
        if constexpr (MODE == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        else if constexpr (MODE == 3) __threadfence();
        sum_partials<MODE == 4>(part + (int64_t)grp * G * kHandoffFloats, out + (int64_t)grp * kHandoffFloats, G);
        if (threadIdx.x == 0) __hip_atomic_store(tickets + grp, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ __launch_bounds__(kHandoffThreads) void handoff_reduce_kernel(float* part, float* __restrict__ out, int G) {
    sum_partials<false>(part + (int64_t)blockIdx.x * G * kHandoffFloats, out + (int64_t)blockIdx.x * kHandoffFloats, G);
}

// Grid barrier probe: N resident workgroups of 512 threads pass `rounds` barriers. MODE:
//   0: one counter: thread 0 adds 1, then polls it until it reaches (r + 1) N;
//   1: one flag per workgroup: thread 0 stores r + 1 to its flag, wave 0 polls every flag (lane l
//      flags l, l + 64, ...) until all hold at least r + 1;
//   2: 8 counters: thread 0 adds 1 to counter w % 8, lanes 0-7 each poll one counter until it holds
//      (r + 1) times its workgroups;
//   3: as 2, and each workgroup hands over 1 KiB per round: wave 0 stores it device-coherent before
//      arriving, and after the barrier reads, device-coherent, what workgroup (w + 1) % N stored;
//   4: as 3 with plain stores and loads, an agent-scope release fence before arriving and an
//      acquire fence after the barrier.
// Hand-off words of round r from workgroup w hold r N + w + 1 (double-buffered by round parity: a
// slot is rewritten two rounds later, after its reader has passed the barrier between); a mismatch
// sets err bit 2.
constexpr int kBarrierThreads = 512;

template <int MODE>
__global__ __launch_bounds__(kBarrierThreads) void barrier_kernel(int32_t* sync, int32_t* hand, int rounds,
                                                                 int32_t* err) {
    const int wg = blockIdx.x, N = gridDim.x, tid = threadIdx.x;
    bool ok = true;  // this thread has not timed out (after a time-out it waits no more)
    for (int r = 0; r < rounds; ++r) {
        if constexpr (MODE >= 3) {
            if (tid < 64) {
                const uint32_t v = (uint32_t)(r * N + wg + 1);
                int32_t* dst = hand + ((int64_t)(r & 1) * N + wg) * 256 + tid * 4;
                if constexpr (MODE == 3) {
                    store_coherent(dst, uint4{v, v, v, v});
                    __builtin_amdgcn_s_waitcnt(0);
                } else {
                    *reinterpret_cast<uint4*>(dst) = uint4{v, v, v, v};
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
                }
            }
        }
        if (MODE == 1) {
            if (tid == 0) __hip_atomic_store(sync + kFlagWords + wg, r + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (tid == 0) {
            __hip_atomic_fetch_add(sync + (MODE == 0 ? 0 : wg % kCounters), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // A wait that gives up sets err bit 1 once; that thread waits no more.
        if (MODE == 0) {
            if (tid == 0 && ok && !poll_at_least(sync, (r + 1) * N)) {
                ok = false;
                atomicOr(err, 1);
            }
        } else if (MODE == 1) {
            if (tid < 64 && ok) {
                for (int polls = 0;; ++polls) {
                    bool mine = true;
                    for (int f = tid; f < N; f += 64)
                        mine &= __hip_atomic_load(sync + kFlagWords + f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > r;
                    if (__all(mine)) break;
                    if (polls >= kSpinLimit) {
                        ok = false;
                        if (tid == 0) atomicOr(err, 1);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        } else {
            if (tid < kCounters && ok && !poll_at_least(sync + tid, (r + 1) * counter_members(tid, N))) {
                ok = false;
                atomicOr(err, 1);
            }
        }
        __syncthreads();
        if constexpr (MODE >= 3) {
            if (tid < 64) {
                const int src = wg + 1 < N ? wg + 1 : 0;
                int32_t* from = hand + ((int64_t)(r & 1) * N + src) * 256 + tid * 4;
                uint4 u;
                if constexpr (MODE == 3) {
                    u = load_coherent(from);
                } else {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    u = *reinterpret_cast<const uint4*>(from);
                }
                const uint32_t want = (uint32_t)(r * N + src + 1);
                if (u.x != want || u.y != want || u.z != want || u.w != want) atomicOr(err, 2);
            }
        }
    }
    finish_and_clear(sync, MODE == 1 ? N : 0);
}

// Phase-chain probe: phase p of workgroup w streams chunks 16-byte chunks of src from chunk
// (p N + w) chunks on (non-temporal) and hands 1 KiB to phase p + 1, which reads what workgroup
// (w + 1) % N wrote (it must hold p + 1: phase p writes what it read plus one, phase 0 writes 1; a
// mismatch sets err bit 2). A phase first issues up to kChainPre loads per thread (at most 128 KiB
// per workgroup), then streams the rest 4 loads in flight per thread. PERSISTENT = false runs phases
// [phase0, phase0 + phases) with plain hand-off stores and loads: one phase per launch is the
// graph of kernels. PERSISTENT = true runs every phase in one launch of resident workgroups:
// phase p's first loads are in flight while it waits for every arrival of phase p - 1 (the
// 8-counter barrier with device-coherent hand-off stores and loads), and it arrives after its
// hand-off store.
constexpr int kChainThreads = 512, kChainU = 4, kChainPre = 16;

template <bool PERSISTENT>
__global__ __launch_bounds__(kChainThreads) void chain_kernel(const u32x4v* __restrict__ src, int64_t chunks,
                                                             int phase0, int phases, int32_t* sync, int32_t* hand,
                                                             int32_t* err, int32_t* sink) {
    const int wg = blockIdx.x, N = gridDim.x, tid = threadIdx.x;
    const int from_wg = wg + 1 < N ? wg + 1 : 0;
    uint32_t acc = 0;
    bool ok = true;
    for (int p = phase0; p < phase0 + phases; ++p) {
        const u32x4v* s = src + ((int64_t)p * N + wg) * chunks;
        u32x4v pre[kChainPre];
#pragma unroll
        for (int u = 0; u < kChainPre; ++u) {
            const int64_t i = tid + (int64_t)u * kChainThreads;
            pre[u] = i < chunks ? __builtin_nontemporal_load(s + i) : u32x4v{0u, 0u, 0u, 0u};
        }
        uint32_t in = 0;
        if (p > 0) {
            if constexpr (PERSISTENT) {
                if (tid < kCounters && ok && !poll_at_least(sync + tid, p * counter_members(tid, N))) {
                    ok = false;
                    atomicOr(err, 1);
                }
                __syncthreads();
            }
            if (tid < 64) {
                int32_t* from = hand + ((int64_t)((p - 1) & 1) * N + from_wg) * 256 + tid * 4;
                const uint4 u = PERSISTENT ? load_coherent(from) : *reinterpret_cast<const uint4*>(from);
                if (u.x != (uint32_t)p || u.y != (uint32_t)p || u.z != (uint32_t)p || u.w != (uint32_t)p)
                    atomicOr(err, 2);
                in = u.x;
            }
        }
#pragma unroll
        for (int u = 0; u < kChainPre; ++u) acc ^= pre[u].x ^ pre[u].y ^ pre[u].z ^ pre[u].w;
        for (int64_t i0 = tid + (int64_t)kChainThreads * kChainPre; i0 < chunks; i0 += (int64_t)kChainThreads * kChainU) {
            u32x4v v[kChainU];
#pragma unroll
            for (int u = 0; u < kChainU; ++u) {
                const int64_t i = i0 + (int64_t)u * kChainThreads;
                v[u] = __builtin_nontemporal_load(s + (i < chunks ? i : chunks - 1));
            }
#pragma unroll
            for (int u = 0; u < kChainU; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
        if (tid < 64) {
            const uint32_t o = in + 1;
            int32_t* dst = hand + ((int64_t)(p & 1) * N + wg) * 256 + tid * 4;
            if constexpr (PERSISTENT) {
                store_coherent(dst, uint4{o, o, o, o});
                __builtin_amdgcn_s_waitcnt(0);
            } else {
                *reinterpret_cast<uint4*>(dst) = uint4{o, o, o, o};
            }
        }
        if constexpr (PERSISTENT) {
            if (tid == 0) __hip_atomic_fetch_add(sync + wg % kCounters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (acc == 0x9e3779b9u) sink[0] = (int32_t)acc;
    if constexpr (PERSISTENT) finish_and_clear(sync, 0);
}

// Workgroups of `kernel` (at `threads` threads) that fit on the current device at once.
template <typename K>
static int resident_workgroups(K kernel, int threads) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess)
        return 0;
    return cus * per_cu;
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

extern "C" int mx_handoff_probe(float* part, int64_t part_bytes, float* out, int64_t out_bytes, int32_t* tickets,
                                int64_t tickets_bytes, int32_t workgroups, int32_t group, int32_t mode, void* stream) {
    const char* what = "mx_handoff_probe";
    clear_error();
    if (mode < 0 || mode > 4) return fail(MX_ERR_INVALID, "%s: mode must be 0 to 4", what);
    if (workgroups <= 0 || group <= 0 || workgroups % group || workgroups > (1 << 20))
        return fail(MX_ERR_INVALID, "%s: need 0 < workgroups <= 2^20, a multiple of group > 0", what);
    const int groups = workgroups / group;
    const int64_t per = (int64_t)probe::kHandoffFloats * sizeof(float);
    if (!part || (mode > 0 && !out) || (mode > 1 && !tickets)) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (part_bytes < workgroups * per || (mode > 0 && out_bytes < groups * per) ||
        (mode > 1 && tickets_bytes < groups * (int64_t)sizeof(int32_t)))
        return fail(MX_ERR_INVALID, "%s: buffers need %lld bytes of partials, %lld of sums and %d tickets", what,
                    (long long)(workgroups * per), (long long)(groups * per), groups);
    if (!aligned(part, 16) || (out && !aligned(out, 16)) || (tickets && !aligned(tickets, 4)))
        return fail(MX_ERR_ALIGNMENT, "%s: part and out must be 16-byte aligned", what);
    hipStream_t st = as_stream(stream);
    const dim3 grid(workgroups), block(probe::kHandoffThreads);
    switch (mode) {
        case 0: hipLaunchKernelGGL(probe::handoff_kernel<0>, grid, block, 0, st, part, out, tickets, group); break;
        case 1:
            hipLaunchKernelGGL(probe::handoff_kernel<0>, grid, block, 0, st, part, out, tickets, group);
            hipLaunchKernelGGL(probe::handoff_reduce_kernel, dim3(groups), block, 0, st, part, out, group);
            break;
        case 2: hipLaunchKernelGGL(probe::handoff_kernel<2>, grid, block, 0, st, part, out, tickets, group); break;
        case 3: hipLaunchKernelGGL(probe::handoff_kernel<3>, grid, block, 0, st, part, out, tickets, group); break;
        default: hipLaunchKernelGGL(probe::handoff_kernel<4>, grid, block, 0, st, part, out, tickets, group); break;
    }
    return check_launch(what);
}

extern "C" int mx_barrier_probe(int32_t* sync, int64_t sync_bytes, int32_t* hand, int64_t hand_bytes,
                                int32_t workgroups, int32_t rounds, int32_t mode, int32_t* err, void* stream) {
    const char* what = "mx_barrier_probe";
    clear_error();
    if (mode < 0 || mode > 4) return fail(MX_ERR_INVALID, "%s: mode must be 0 to 4", what);
    if (!sync || !err || (mode >= 3 && !hand)) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (workgroups <= 0 || workgroups > 8192 || rounds < 0 || rounds > 100000)
        return fail(MX_ERR_INVALID, "%s: need 0 < workgroups <= 8192 and 0 <= rounds <= 100000", what);
    if (sync_bytes < (int64_t)(probe::kFlagWords + workgroups) * 4 ||
        (mode >= 3 && hand_bytes < (int64_t)workgroups * 2 * 1024))
        return fail(MX_ERR_INVALID, "%s: sync needs %d words, hand %lld bytes", what, probe::kFlagWords + workgroups,
                    (long long)workgroups * 2 * 1024);
    if (!aligned(sync, 4) || (hand && !aligned(hand, 16))) return fail(MX_ERR_ALIGNMENT, "%s: hand must be 16-byte aligned", what);
    int resident = 0;
    switch (mode) {
        case 0: resident = probe::resident_workgroups(probe::barrier_kernel<0>, probe::kBarrierThreads); break;
        case 1: resident = probe::resident_workgroups(probe::barrier_kernel<1>, probe::kBarrierThreads); break;
        case 2: resident = probe::resident_workgroups(probe::barrier_kernel<2>, probe::kBarrierThreads); break;
        case 3: resident = probe::resident_workgroups(probe::barrier_kernel<3>, probe::kBarrierThreads); break;
        default: resident = probe::resident_workgroups(probe::barrier_kernel<4>, probe::kBarrierThreads); break;
    }
    if (workgroups > resident)
        return fail(MX_ERR_UNSUPPORTED, "%s: %d workgroups, but only %d fit on the device at once", what, workgroups,
                    resident);
    hipStream_t st = as_stream(stream);
    const dim3 grid(workgroups), block(probe::kBarrierThreads);
    switch (mode) {
        case 0: hipLaunchKernelGGL(probe::barrier_kernel<0>, grid, block, 0, st, sync, hand, rounds, err); break;
        case 1: hipLaunchKernelGGL(probe::barrier_kernel<1>, grid, block, 0, st, sync, hand, rounds, err); break;
        case 2: hipLaunchKernelGGL(probe::barrier_kernel<2>, grid, block, 0, st, sync, hand, rounds, err); break;
        case 3: hipLaunchKernelGGL(probe::barrier_kernel<3>, grid, block, 0, st, sync, hand, rounds, err); break;
        default: hipLaunchKernelGGL(probe::barrier_kernel<4>, grid, block, 0, st, sync, hand, rounds, err); break;
    }
    return check_launch(what);
}

extern "C" int mx_chain_probe(const void* src, int64_t src_bytes, int64_t bytes_per_wg, int32_t workgroups,
                              int32_t phase0, int32_t phases, int32_t persistent, int32_t* sync, int64_t sync_bytes,
                              int32_t* hand, int64_t hand_bytes, int32_t* err, int32_t* sink, void* stream) {
    const char* what = "mx_chain_probe";
    clear_error();
    if (!src || !hand || !err || !sink || (persistent && !sync)) return fail(MX_ERR_NULL, "%s: null pointer", what);
    if (workgroups <= 0 || workgroups > 8192 || phases <= 0 || phase0 < 0 || phase0 + phases > 100000 ||
        bytes_per_wg <= 0 || bytes_per_wg % 16)
        return fail(MX_ERR_INVALID, "%s: need 0 < workgroups <= 8192, phases > 0, phase0 >= 0 and 16-byte multiples",
                    what);
    if (persistent && phase0 != 0) return fail(MX_ERR_INVALID, "%s: a persistent launch starts at phase 0", what);
    if ((int64_t)(phase0 + phases) * workgroups * bytes_per_wg > src_bytes)
        return fail(MX_ERR_INVALID, "%s: %d phases x %d x %lld bytes exceed the %lld-byte buffer", what, phase0 + phases,
                    workgroups, (long long)bytes_per_wg, (long long)src_bytes);
    if (hand_bytes < (int64_t)workgroups * 2 * 1024 || (persistent && sync_bytes < (probe::kDoneWord + 1) * 4))
        return fail(MX_ERR_INVALID, "%s: hand needs %lld bytes, sync %d words", what, (long long)workgroups * 2 * 1024,
                    probe::kDoneWord + 1);
    if (!aligned(src, 16) || !aligned(hand, 16)) return fail(MX_ERR_ALIGNMENT, "%s: src and hand must be 16-byte aligned", what);
    hipStream_t st = as_stream(stream);
    const auto* s = static_cast<const probe::u32x4v*>(src);
    const int64_t chunks = bytes_per_wg / 16;
    const dim3 grid(workgroups), block(probe::kChainThreads);
    if (persistent) {
        const int resident = probe::resident_workgroups(probe::chain_kernel<true>, probe::kChainThreads);
        if (workgroups > resident)
            return fail(MX_ERR_UNSUPPORTED, "%s: %d workgroups, but only %d fit on the device at once", what,
                        workgroups, resident);
        hipLaunchKernelGGL(probe::chain_kernel<true>, grid, block, 0, st, s, chunks, 0, phases, sync, hand, err, sink);
    } else {
        hipLaunchKernelGGL(probe::chain_kernel<false>, grid, block, 0, st, s, chunks, phase0, phases, sync, hand, err,
                           sink);
    }
    return check_launch(what);
}
