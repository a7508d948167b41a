// Int8 weight tiles shared by the W8A16 kernels: the packed tile geometry, the
// in-register dequant and the per-wave load pipeline (see w8a16.hip for the layout).
#pragma once

#include "common.h"

namespace mx {
namespace w8a16 {

constexpr int kTileN = 16;
constexpr int kTileK = 64;
constexpr uint32_t kMagic = 0x64646464u;
constexpr uint32_t kSelLo = 0x04010400u;  // bytes 0,1 -> fp16 pair (0x64:b0, 0x64:b1)
constexpr uint32_t kSelHi = 0x04030402u;  // bytes 2,3 -> fp16 pair (0x64:b2, 0x64:b3)

struct U32x4 {
    uint32_t a, b, c, d;
};

// One lane's 16 bytes of a weight tile. Weights are read once per decode step, so the
// loads take the streaming (non-temporal) cache policy; x, which every workgroup re-reads
// from L2, keeps the default one. Measured in the decode step at batch 32: lm_head
// 91.3 -> 82.8 us (6.45 TB/s), qkv 13.1 -> 12.6 us, the step 4.42 -> 4.39 ms.
// STREAM = false where two waves read each tile (the M-split shape): there the default
// policy measured faster (M = 128: qkv 26.1 -> 22.4 us, o 25.1 -> 21.4 us).
#ifndef MX_W8A16_NT_WEIGHTS
#define MX_W8A16_NT_WEIGHTS 1
#endif
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
template <bool STREAM = true>
__device__ __forceinline__ uint4 load_wtile(const uint4* p) {
    if constexpr (MX_W8A16_NT_WEIGHTS && STREAM) {
        const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
        return uint4{v.x, v.y, v.z, v.w};
    } else {
        return *p;
    }
}

// 8 biased bytes (two dwords) -> 8 exact fp16 weights.
__device__ __forceinline__ half8v dequant8(uint32_t d0, uint32_t d1) {
    const U32x4 raw{__builtin_amdgcn_perm(kMagic, d0, kSelLo), __builtin_amdgcn_perm(kMagic, d0, kSelHi),
                    __builtin_amdgcn_perm(kMagic, d1, kSelLo), __builtin_amdgcn_perm(kMagic, d1, kSelHi)};
    const half8v bias = (_Float16)(-1152.0f);
    return __builtin_bit_cast(half8v, raw) + bias;
}

__device__ __forceinline__ half8v load_half8(const _Float16* p) {
    return __builtin_bit_cast(half8v, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ float dot8(half8v a, half8v b, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 0, 1), __builtin_shufflevector(b, b, 0, 1), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 2, 3), __builtin_shufflevector(b, b, 2, 3), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 4, 5), __builtin_shufflevector(b, b, 4, 5), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 6, 7), __builtin_shufflevector(b, b, 6, 7), acc, false);
    return acc;
}

__device__ __forceinline__ uint16_t f2h_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
__device__ __forceinline__ float h2f(const uint16_t* p, int64_t i) {
    return (float)reinterpret_cast<const _Float16*>(p)[i];
}

// ---------------------------------------------------------------------------
// Per-wave software pipeline. A wave owns the k-tiles kt = wave + j*WAVES,
// j < nj, of the workgroup's n-tiles. Stage s of P holds the weight tiles and
// the x fragments of one k-tile; the loads for k-tile j+P are issued as soon
// as k-tile j has been consumed, so P k-tiles (P*NPW KiB of weights plus their
// x fragments) stay in flight per wave.
//
// Every load is issued unconditionally: past the last k-tile the index is
// clamped (the reload hits L2), and x rows past M read row M-1 (MFMA rows are
// independent, those C rows are discarded). With no loads under a branch the
// compiler can wait for exactly the oldest stage (s_waitcnt vmcnt(N)) instead
// of draining every load in flight. Addresses are a wave-uniform base plus a
// fixed 32-bit lane offset.
// ---------------------------------------------------------------------------
// The stage loop shared by both kernels. Prologue: stages 0..P-1 (indices
// clamped when nj < P). Full rounds issue the loads of tile j+P right after
// tile j is consumed, unconditionally. The last round and a half issue only
// the loads still in range, then drain.
#define PIPELINE_BODY(P, nj, st, load, COMPUTE) PIPELINE_BODY_HOOK(P, nj, st, load, COMPUTE, (void)0)

// HOOK runs once, after the first P stages' loads are issued and before the first compute:
// loads it issues overlap the pipeline's first round trip.
#define PIPELINE_BODY_HOOK(P, nj, st, load, COMPUTE, HOOK)         \
    _Pragma("unroll") for (int s = 0; s < P; ++s) load(s, st[s]); \
    HOOK;                                                           \
    PIPELINE_REST(P, nj, st, load, COMPUTE)

// Everything after the prologue: for callers that issue the first P stages themselves.
#define PIPELINE_REST(P, nj, st, load, COMPUTE)                     \
    int j0 = 0;                                                     \
    for (; j0 + 2 * P <= nj; j0 += P) {                             \
        _Pragma("unroll") for (int s = 0; s < P; ++s) {             \
            COMPUTE;                                                \
            load(j0 + s + P, st[s]);                                \
        }                                                           \
    }                                                               \
    _Pragma("unroll") for (int s = 0; s < P; ++s) {                 \
        if (j0 + s < nj) {                                          \
            COMPUTE;                                                \
            if (j0 + s + P < nj) load(j0 + s + P, st[s]);           \
        }                                                           \
    }                                                               \
    _Pragma("unroll") for (int s = 0; s < P; ++s) {                 \
        if (j0 + P + s < nj) { COMPUTE; }                           \
    }

}  // namespace w8a16
}  // namespace mx
