// Measurement tool (libmbs_probe.so, not the GEMM library): a plain streaming
// read of a device buffer with 16-byte non-temporal loads, the floor a
// memory-bound decode GEMM is compared against.  Each thread keeps U loads in
// flight (grid-stride over 16-byte chunks) and folds them into one word; the
// words of a wave are combined and lane 0 writes one per wave, so no load can
// be dropped as dead code and the writes are 4 bytes per 64 lanes.
#include "mxfp4_device.h"
#include "mbs_probe.h"

namespace mbs {

template <int U>
__global__ void __launch_bounds__(256) stream_read_kernel(const uint8_t* __restrict__ src, uint32_t n16,
                                                          uint32_t* __restrict__ sink)
{
    const rsrc_t r = make_rsrc(src, n16 * 16u);
    const uint32_t stride = gridDim.x * 256u;
    uint32_t x = 0;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n16; i += stride * U) {
        i32x4 v[U];
        static_for<U>([&](auto u) {
            const uint32_t idx = i + (uint32_t)u * stride;
            v[u] = load16nt(r, idx < n16 ? idx * 16u : kOOB);
        });
        static_for<U>([&](auto u) { x ^= (uint32_t)(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]); });
    }
    for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

}  // namespace mbs

using namespace mbs;

extern "C" int mbs_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int grid,
                                     void* stream)
{
    if (!src || !sink || grid < 1 || grid > 65535 || bytes % 16 || bytes == 0 ||
        bytes >= ((size_t)1 << 31) || reinterpret_cast<uintptr_t>(src) % 16)
        return 1;
    (void)hipGetLastError();
    hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t*>(src), (uint32_t)(bytes / 16), sink);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}
