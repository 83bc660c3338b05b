// floors.hip — measurement kernels for the decode layer's floors (not part of
// the drop-in ABI; built into libtsugumi_floors.so, loaded by bench.py
// --floors only).
//
//  * floor_empty_kernel: the one-launch decode layer's grid (256 blocks) and
//    block size with the same dynamic LDS, doing nothing: back-to-back in a
//    HIP graph its period is the launch-to-launch floor of any one-launch
//    layer of that shape.
//  * floor_stream_kernel: the same grid reading the routed experts' bytes
//    (8 expert blobs at given ids, `payload` bytes each) once, with 16-byte
//    nontemporal loads all in flight, the way the layer's weight phase reads
//    them, and nothing else: the time to move a decode layer's expert bytes
//    when the routing is known at launch.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

__global__ void floor_empty_kernel(uint32_t* sink, uint32_t magic) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (threadIdx.x == 0 && blockIdx.x == magic) sink[0] = smem[0];
}

struct StreamArgs {
    const uint8_t* base;
    uint64_t stride;
    uint32_t ids[8];
    uint32_t payload;  // bytes per expert, a multiple of 16
    uint32_t* sink;
    uint32_t magic;
};

// Block b reads 1/32 of slot b % 8's blob (a contiguous run), 16 bytes per
// lane per step, every load of a lane issued before any is used.
__global__ __launch_bounds__(1024) void floor_stream_kernel(StreamArgs a) {
    const uint32_t slot = blockIdx.x % 8u, member = blockIdx.x / 8u;
    const uint32_t members = gridDim.x / 8u;
    const uint32_t chunks = a.payload / 16u;
    const uint32_t per = (chunks + members - 1u) / members;
    const uint32_t c0 = member * per, c1 = min(c0 + per, chunks);
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t* p = reinterpret_cast<const u32x4_t*>(a.base + (uint64_t)a.ids[slot] * a.stride);
    constexpr int kInFlight = 8;
    uint32_t acc = 0;
    for (uint32_t c = c0 + threadIdx.x; c < c1; c += blockDim.x * kInFlight) {
        u32x4_t v[kInFlight];
#pragma unroll
        for (int i = 0; i < kInFlight; ++i) {
            const uint32_t cc = c + i * blockDim.x;
            v[i] = cc < c1 ? __builtin_nontemporal_load(p + cc) : u32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < kInFlight; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == a.magic) a.sink[blockIdx.x] = acc;  // keeps the loads; practically never taken
}

}  // namespace

extern "C" int tsg_floor_empty(void* stream, uint32_t blocks, uint32_t threads, uint32_t lds,
                               uint32_t* sink) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(floor_empty_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return 1;
    hipLaunchKernelGGL(floor_empty_kernel, dim3(blocks), dim3(threads), lds,
                       reinterpret_cast<hipStream_t>(stream), sink, 0xFFFFFFFFu);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

extern "C" int tsg_floor_stream(void* stream, const void* base, uint64_t stride,
                                const uint32_t* ids8, uint32_t payload, uint32_t blocks,
                                uint32_t threads, uint32_t* sink) {
    if (payload % 16 || blocks % 8 || !base || !ids8 || !sink) return 1;
    StreamArgs a{};
    a.base = static_cast<const uint8_t*>(base);
    a.stride = stride;
    for (int i = 0; i < 8; ++i) a.ids[i] = ids8[i];
    a.payload = payload;
    a.sink = sink;
    a.magic = 0x9E3779B9u;
    hipLaunchKernelGGL(floor_stream_kernel, dim3(blocks), dim3(threads), 0,
                       reinterpret_cast<hipStream_t>(stream), a);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
