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
