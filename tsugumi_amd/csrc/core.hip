// core.hip — context, errors, HBM-resident layers and synthetic generators.
#include "tsg_internal.hpp"

#include <cstring>
#include <new>

namespace tsg {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

tsg_status fail(tsg_status status, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

tsg_status check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TSG_ERR_HIP, "%s launch: %s", what, hipGetErrorString(e));
    return TSG_OK;
}

}  // namespace tsg

using namespace tsg;

extern "C" const char* tsg_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* tsg_version(void) { return "0.1.0"; }

extern "C" const char* tsg_status_string(tsg_status s) {
    switch (s) {
        case TSG_OK: return "ok";
        case TSG_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TSG_ERR_ALIGNMENT: return "misaligned pointer or offset";
        case TSG_ERR_UNSUPPORTED: return "unsupported configuration";
        case TSG_ERR_DECLINED: return "declined";
        case TSG_ERR_HIP: return "HIP runtime error";
        case TSG_ERR_OUT_OF_MEMORY: return "out of device memory";
        case TSG_ERR_FORMAT: return "invalid MoEPack install";
        case TSG_ERR_IO: return "MoEPack file missing or unreadable";
        case TSG_ERR_GROUPING_INVALID_QUERY_COUNT: return "invalidQueryCount";
        case TSG_ERR_GROUPING_INVALID_TOP_K: return "invalidTopK";
        case TSG_ERR_GROUPING_INVALID_NUM_EXPERTS: return "invalidNumExperts";
        case TSG_ERR_GROUPING_INVALID_TILE_EXPERT_COUNT: return "invalidTileExpertCount";
        case TSG_ERR_GROUPING_PAIR_COUNT_MISMATCH: return "pairCountMismatch";
        case TSG_ERR_GROUPING_TOKEN_OUT_OF_RANGE: return "tokenOutOfRange";
        case TSG_ERR_GROUPING_RANK_OUT_OF_RANGE: return "rankOutOfRange";
        case TSG_ERR_GROUPING_EXPERT_OUT_OF_RANGE: return "expertOutOfRange";
        case TSG_ERR_GROUPING_DUPLICATE_TOKEN_RANK: return "duplicateTokenRank";
        case TSG_ERR_GROUPING_SORT_KEY_COUNT_MISMATCH: return "expertSortKeyCountMismatch";
    }
    return "unknown status";
}

// ------------------------------------------------------------------ context

extern "C" tsg_status tsg_ctx_create(int device, tsg_ctx** out) {
    TSG_REQUIRE(out != nullptr, TSG_ERR_INVALID_ARGUMENT, "out is NULL");
    *out = nullptr;
    int count = 0;
    TSG_HIP_TRY(hipGetDeviceCount(&count));
    TSG_REQUIRE(device >= 0 && device < count, TSG_ERR_INVALID_ARGUMENT,
                "device %d out of range (%d devices)", device, count);
    // the context's set-up runs with `device` current; the caller's current
    // device is restored on every return
    int prev = 0;
    TSG_HIP_TRY(hipGetDevice(&prev));
    struct Restore {
        int dev;
        ~Restore() { (void)hipSetDevice(dev); }
    } restore{prev};
    TSG_HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    TSG_HIP_TRY(hipGetDeviceProperties(&prop, device));
    TSG_REQUIRE(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0, TSG_ERR_UNSUPPORTED,
                "device %d is %s; this library is built for gfx950 (MI355X) only", device,
                prop.gcnArchName);
    tsg_ctx* ctx = new (std::nothrow) tsg_ctx();
    TSG_REQUIRE(ctx != nullptr, TSG_ERR_OUT_OF_MEMORY, "host allocation failed");
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    // The fused grouped GEMM keeps every item of a routed block on one XCD
    // (one queue per XCD); an XCD count it cannot map one to one onto its
    // queues (unknown, not a power of two, more than kMaxGemmQueues) leaves
    // the fused launch off (gemm_queues = 0) and the two-launch form runs.
    int n_xcc = 0;
    if (hipDeviceGetAttribute(&n_xcc, hipDeviceAttributeNumberOfXccs, device) != hipSuccess)
        n_xcc = 0;
    ctx->gemm_queues = n_xcc > 0 && (uint32_t)n_xcc <= kMaxGemmQueues && (n_xcc & (n_xcc - 1)) == 0
                           ? (uint32_t)n_xcc
                           : 0u;
    hipError_t e = hipMalloc(&ctx->counters, sizeof(uint32_t) * kMaxCounters);
    if (e == hipSuccess)
        e = hipMalloc(&ctx->logits, sizeof(float) * kMaxPromptRows * kMaxExperts);
    if (e == hipSuccess)
        e = hipMalloc(&ctx->act_replicas, sizeof(uint16_t) * kActReplicas * kActReplicaHalves);
    if (e == hipSuccess) e = hipMalloc(&ctx->verify_words, sizeof(uint64_t) * kVerifyWords);
    if (e == hipSuccess) e = hipMalloc(&ctx->gemm_sched, sizeof(uint32_t) * kGemmSchedWords);
    if (e == hipSuccess) e = hipMemset(ctx->gemm_sched, 0, sizeof(uint32_t) * kGemmSchedWords);
    if (e == hipSuccess) e = hipMemset(ctx->counters, 0, sizeof(uint32_t) * kMaxCounters);
    // The one-launch decode layer's hand-off words carry the launch's tag
    // (epoch + 1, never 0) and the epoch starts at 0 here: words left by an
    // earlier context in recycled memory would carry tags this context will
    // issue again, so the regions start at tag 0.
    if (e == hipSuccess)
        e = hipMemset(ctx->act_replicas, 0, sizeof(uint16_t) * kActReplicas * kActReplicaHalves);
    if (e == hipSuccess) e = hipMemset(ctx->verify_words, 0, sizeof(uint64_t) * kVerifyWords);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    // this device's address of the no-alloc grouping scratch (device current)
    const tsg_status st = e == hipSuccess ? group_noalloc_setup(ctx) : TSG_OK;
    if (e != hipSuccess || st != TSG_OK) {
        (void)hipFree(ctx->counters);
        (void)hipFree(ctx->logits);
        (void)hipFree(ctx->act_replicas);
        (void)hipFree(ctx->verify_words);
        (void)hipFree(ctx->gemm_sched);
        delete ctx;
        if (st != TSG_OK) return st;
        return fail(TSG_ERR_OUT_OF_MEMORY, "context scratch: %s", hipGetErrorString(e));
    }
    *out = ctx;
    return TSG_OK;
}

extern "C" void tsg_ctx_destroy(tsg_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(ctx->counters);
    (void)hipFree(ctx->logits);
    (void)hipFree(ctx->act_replicas);
    (void)hipFree(ctx->verify_words);
    (void)hipFree(ctx->gemm_sched);
    delete ctx;
}

extern "C" tsg_status tsg_ctx_set_affine_group_size(tsg_ctx* ctx, uint32_t g) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(group_ok(g), TSG_ERR_INVALID_ARGUMENT,
                "unsupported affine group size %u (supported: 32, 64)", g);
    ctx->group_size = g;
    return TSG_OK;
}

extern "C" tsg_status tsg_ctx_set_affine_scheme(tsg_ctx* ctx, tsg_affine_scheme scheme) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_REQUIRE(scheme == TSG_AFFINE || scheme == TSG_SYM, TSG_ERR_INVALID_ARGUMENT,
                "unknown affine scheme %d", (int)scheme);
    ctx->scheme = scheme;
    return TSG_OK;
}

extern "C" tsg_status tsg_ctx_synchronize(tsg_ctx* ctx, tsg_stream stream) {
    TSG_REQUIRE(ctx, TSG_ERR_INVALID_ARGUMENT, "ctx is NULL");
    TSG_HIP_TRY(hipStreamSynchronize(as_stream(stream)));
    // Kernels that detect an error on the device set a bit of this word (the
    // one-launch decode layer on a hand-off timeout, the device grouping on
    // an out-of-range expert id or an overfull work list, the device-list rows
    // path on a block it cannot take); the outputs of the affected launches
    // are invalid. Reading clears it.
    uint32_t err = 0;
    TSG_HIP_TRY(hipMemcpy(&err, ctx->counters + kSyncErrorWord, sizeof(err),
                          hipMemcpyDeviceToHost));
    if (err) {
        TSG_HIP_TRY(hipMemset(ctx->counters + kSyncErrorWord, 0, sizeof(err)));
        if (err & kErrGroupExpertRange)
            return fail(TSG_ERR_GROUPING_EXPERT_OUT_OF_RANGE,
                        "expertOutOfRange: the device grouping met a route expert id >= "
                        "numExperts; those pairs were not grouped");
        if (err & kErrGroupBlocks)
            return fail(TSG_ERR_INVALID_ARGUMENT,
                        "the device grouping's work list exceeded max_blocks");
        if (err & kErrRowsBlock)
            return fail(TSG_ERR_INVALID_ARGUMENT,
                        "rows path: a device block had no rows, more than 8, or an expert past "
                        "the layer; it was skipped");
        if (err & kErrVerifyRouting)
            return fail(TSG_ERR_INVALID_ARGUMENT,
                        "verify layer: a token had fewer than 8 eligible router logits (NaN or "
                        "-inf scores); the layer's outputs are NaN");
        if (err & kErrRouterWait)
            return fail(TSG_ERR_HIP, "staged router: the selecting block timed out waiting for "
                                     "the other blocks' logits; the routing is invalid");
        if (err & kErrGemmBlock)
            return fail(TSG_ERR_INVALID_ARGUMENT,
                        "grouped GEMM: a routed block named an expert past the layer; it was "
                        "skipped and its rows were not written");
        if (err & kErrGemmWait)
            return fail(TSG_ERR_HIP, "fused grouped GEMM: a down item timed out waiting for its "
                                     "block's gate/up tiles, or an XCD queue was not drained; "
                                     "the layer's outputs are invalid");
        return fail(TSG_ERR_HIP, "fused decode layer: a block timed out waiting for the "
                                 "others; outputs of the affected launch are invalid");
    }
    return TSG_OK;
}

// ---------------------------------------------------------------- layers

static tsg_status check_offsets(const tsg_expert_offsets* o, uint64_t stride) {
    TSG_REQUIRE(o != nullptr, TSG_ERR_INVALID_ARGUMENT, "offsets is NULL");
    const uint32_t* v = &o->gate_w;
    for (int i = 0; i < 9; ++i) {
        TSG_REQUIRE(v[i] < stride, TSG_ERR_INVALID_ARGUMENT,
                    "sub-tensor offset %u lies outside the %llu-byte expert stride", v[i],
                    (unsigned long long)stride);
        // the reference's contract: sub-tensors on 2 bytes (DequantInt4GEMV.swift:93-96)
        TSG_REQUIRE(v[i] % 2 == 0, TSG_ERR_ALIGNMENT,
                    "sub-tensor offset %u is not 2-byte aligned", v[i]);
    }
    TSG_REQUIRE(stride % 2 == 0, TSG_ERR_ALIGNMENT, "expert stride must be even");
    return TSG_OK;
}

// Whether the kernels can read a layer file's blobs where they lie: weights
// are read as 16-byte chunks, scale and bias windows as dwords, experts on
// 16-byte strides. The shipped sym/g32 layouts always are; the reference
// only promises 2-byte sub-tensors.
static bool kernel_aligned(const tsg_expert_offsets& o, uint64_t stride) {
    return o.gate_w % 16 == 0 && o.up_w % 16 == 0 && o.down_w % 16 == 0 &&
           ((o.gate_s | o.up_s | o.down_s | o.gate_b | o.up_b | o.down_b) % 4) == 0 &&
           stride % 16 == 0;
}

// A new layout of a blob whose sub-tensors are off the kernels' alignment:
// each distinct sub-tensor offset starts a run that reaches to the next one
// (the last to the end of the blob); runs keep their order and start on 256
// bytes; the stride is rounded up to 16 KiB like the packer's
// (RepackPlanner.swift:514-516). Offsets that alias (sym biases = scales)
// keep aliasing.
static void relayout(tsg_layer* l, const tsg_expert_offsets& fo, uint64_t fstride) {
    const uint32_t* fv = &fo.gate_w;
    uint64_t starts[9];
    uint32_t n = 0;
    for (int i = 0; i < 9; ++i) {
        bool seen = false;
        for (uint32_t j = 0; j < n; ++j) seen = seen || starts[j] == fv[i];
        if (!seen) starts[n++] = fv[i];
    }
    std::sort(starts, starts + n);
    uint64_t cur = 0;
    for (uint32_t j = 0; j < n; ++j) {
        const uint64_t end = j + 1 < n ? starts[j + 1] : fstride;
        cur = (cur + 255u) & ~uint64_t(255u);
        l->segments[j] = tsg_layer_segment{starts[j], end - starts[j], cur};
        cur += end - starts[j];
    }
    l->n_segments = n;
    l->expert_stride = (cur + 16383u) / 16384u * 16384u;
    uint32_t* dv = &l->offsets.gate_w;
    for (int i = 0; i < 9; ++i)
        for (uint32_t j = 0; j < n; ++j)
            if (l->segments[j].file_off == fv[i]) dv[i] = (uint32_t)l->segments[j].dev_off;
}

extern "C" tsg_status tsg_layer_create(tsg_ctx* ctx, uint32_t num_experts, uint64_t stride,
                                       const tsg_expert_offsets* offsets, tsg_layer** out) {
    TSG_REQUIRE(ctx && out, TSG_ERR_INVALID_ARGUMENT, "ctx/out is NULL");
    *out = nullptr;
    TSG_REQUIRE(num_experts > 0 && num_experts <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "num_experts %u not in 1..%u", num_experts, kMaxExperts);
    tsg_status st = check_offsets(offsets, stride);
    if (st != TSG_OK) return st;
    tsg_layer geo;
    geo.file_stride = geo.expert_stride = stride;
    geo.file_offsets = geo.offsets = *offsets;
    if (!kernel_aligned(*offsets, stride)) relayout(&geo, *offsets, stride);
    TSG_REQUIRE(geo.expert_stride <= 0xFFFFFFFFull, TSG_ERR_INVALID_ARGUMENT,
                "expert stride %llu is too large", (unsigned long long)geo.expert_stride);
    TSG_HIP_TRY(hipSetDevice(ctx->device));
    void* base = nullptr;
    const size_t bytes = (size_t)num_experts * geo.expert_stride;
    hipError_t e = hipMalloc(&base, bytes);
    if (e != hipSuccess)
        return fail(TSG_ERR_OUT_OF_MEMORY, "layer of %llu bytes: %s", (unsigned long long)bytes,
                    hipGetErrorString(e));
    tsg_layer* l = new tsg_layer(geo);
    l->ctx = ctx;
    l->base = static_cast<uint8_t*>(base);
    l->owned = true;
    l->num_experts = num_experts;
    *out = l;
    return TSG_OK;
}

extern "C" tsg_status tsg_layer_wrap(tsg_ctx* ctx, void* device_base, uint32_t num_experts,
                                     uint64_t stride, const tsg_expert_offsets* offsets,
                                     tsg_layer** out) {
    TSG_REQUIRE(ctx && out && device_base, TSG_ERR_INVALID_ARGUMENT, "NULL argument");
    *out = nullptr;
    TSG_REQUIRE(num_experts > 0 && num_experts <= kMaxExperts, TSG_ERR_INVALID_ARGUMENT,
                "num_experts %u not in 1..%u", num_experts, kMaxExperts);
    TSG_REQUIRE(reinterpret_cast<uintptr_t>(device_base) % 16 == 0, TSG_ERR_ALIGNMENT,
                "layer base must be 16-byte aligned");
    tsg_status st = check_offsets(offsets, stride);
    if (st != TSG_OK) return st;
    // caller-owned memory holds the file image as it is: it cannot be laid out anew
    TSG_REQUIRE(kernel_aligned(*offsets, stride), TSG_ERR_ALIGNMENT,
                "wrapped HBM is read where it lies, so weight sub-tensors must start on 16 "
                "bytes and scales/biases on 4; tsg_layer_create + tsg_layer_upload re-lay a "
                "2-byte aligned layout");
    tsg_layer* l = new tsg_layer();
    l->ctx = ctx;
    l->base = static_cast<uint8_t*>(device_base);
    l->owned = false;
    l->num_experts = num_experts;
    l->expert_stride = l->file_stride = stride;
    l->offsets = l->file_offsets = *offsets;
    *out = l;
    return TSG_OK;
}

extern "C" tsg_status tsg_layer_upload(tsg_layer* layer, tsg_stream stream, const void* host,
                                       uint64_t nbytes, uint64_t dst_offset) {
    TSG_REQUIRE(layer && host, TSG_ERR_INVALID_ARGUMENT, "NULL argument");
    const uint64_t fs = layer->file_stride;
    const uint64_t total = (uint64_t)layer->num_experts * fs;
    TSG_REQUIRE(dst_offset <= total && nbytes <= total - dst_offset, TSG_ERR_INVALID_ARGUMENT,
                "upload of %llu bytes at %llu exceeds the %llu-byte layer",
                (unsigned long long)nbytes, (unsigned long long)dst_offset,
                (unsigned long long)total);
    const hipStream_t hs = as_stream(stream);
    if (layer->n_segments == 0) {
        TSG_HIP_TRY(hipMemcpyAsync(layer->base + dst_offset, host, nbytes, hipMemcpyHostToDevice,
                                   hs));
        return TSG_OK;
    }
    // file bytes [dst_offset, dst_offset + nbytes) -> each run's place in the
    // new layout; bytes outside every run (padding) are not needed
    const uint8_t* src = static_cast<const uint8_t*>(host);
    const uint64_t lo = dst_offset, hi = dst_offset + nbytes;
    for (uint64_t e = lo / fs; e < layer->num_experts && e * fs < hi; ++e) {
        for (uint32_t j = 0; j < layer->n_segments; ++j) {
            const tsg_layer_segment& sg = layer->segments[j];
            const uint64_t a = std::max(lo, e * fs + sg.file_off);
            const uint64_t b = std::min(hi, e * fs + sg.file_off + sg.len);
            if (a >= b) continue;
            uint8_t* dst = layer->base + e * layer->expert_stride + sg.dev_off +
                           (a - (e * fs + sg.file_off));
            TSG_HIP_TRY(hipMemcpyAsync(dst, src + (a - lo), b - a, hipMemcpyHostToDevice, hs));
        }
    }
    return TSG_OK;
}

namespace tsg {
// Geometry of a layer for host code outside this file (the MoEPack loader).
// The layer FILE's geometry (what tsg_layer_upload takes), not the HBM image's.
void layer_geometry(const tsg_layer* layer, int* device, uint32_t* num_experts,
                    uint64_t* expert_stride, tsg_expert_offsets* offsets) {
    *device = layer->ctx->device;
    *num_experts = layer->num_experts;
    *expert_stride = layer->file_stride;
    *offsets = layer->file_offsets;
}
}  // namespace tsg

extern "C" void* tsg_layer_device_ptr(const tsg_layer* layer) {
    return layer ? layer->base : nullptr;
}

extern "C" tsg_status tsg_layer_get_geometry(const tsg_layer* layer, uint64_t* device_stride,
                                             tsg_expert_offsets* device_offsets) {
    TSG_REQUIRE(layer && device_stride && device_offsets, TSG_ERR_INVALID_ARGUMENT,
                "NULL argument");
    *device_stride = layer->expert_stride;
    *device_offsets = layer->offsets;
    return TSG_OK;
}

extern "C" void tsg_layer_destroy(tsg_layer* layer) {
    if (!layer) return;
    if (layer->owned) {
        (void)hipSetDevice(layer->ctx->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(layer->base);
    }
    delete layer;
}

// ------------------------------------------------------------- generators

namespace {

// Output n of the SplitMix64 stream seeded `seed` (SplitMix64.swift:31-37):
// the state after n+1 steps is seed + (n+1) * golden, so any output is one mix.
__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t n) {
    uint64_t z = seed + (n + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// sigma * N(0,1) by Irwin-Hall: the sum of 12 uniforms in [0,1) minus 6,
// summed in order in fp32 (IEEE adds only, so any platform reproduces it).
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    float s = 0.0f;
    for (int k = 0; k < 12; ++k)
        s += (float)(splitmix_at(seed, i * 12 + k) >> 40) * (1.0f / 16777216.0f);
    return s - 6.0f;
}

__global__ void gen_bytes_kernel(uint64_t seed, uint8_t* out, uint64_t n) {
    const uint64_t words = (n + 7) / 8;
    for (uint64_t w = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; w < words;
         w += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t v = splitmix_at(seed, w);
        if (w * 8 + 8 <= n) {
            reinterpret_cast<uint2*>(out)[w] = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
        } else {
            for (uint64_t b = w * 8; b < n; ++b) out[b] = (uint8_t)(v >> (8 * (b - w * 8)));
        }
    }
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
    const uint32_t bits = __float_as_uint(x);
    return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

__global__ void gen_bf16_normal_kernel(uint64_t seed, uint16_t* out, uint64_t n, float sigma,
                                       int abs_value, float divisor) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float v = normal_at(seed, i) * sigma;
        if (abs_value) v = fabsf(v);
        v = v / divisor;
        out[i] = f32_to_bf16_rne(v);
    }
}

__global__ void gen_f16_normal_kernel(uint64_t seed, uint16_t* out, uint64_t n, float sigma) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float v = normal_at(seed, i) * sigma;
        if (fabsf(v) < 7.62939453125e-06f) v = 0.0f;  // 2^-17
        out[i] = f32_to_f16(v);
    }
}

unsigned grid_for(uint64_t items) {
    uint64_t g = (items + 255) / 256;
    if (g > 65536) g = 65536;
    if (g == 0) g = 1;
    return (unsigned)g;
}

}  // namespace

extern "C" tsg_status tsg_gen_bytes(tsg_stream stream, uint64_t seed, uint8_t* out, uint64_t n) {
    TSG_REQUIRE(out || n == 0, TSG_ERR_INVALID_ARGUMENT, "out is NULL");
    TSG_REQUIRE(reinterpret_cast<uintptr_t>(out) % 8 == 0, TSG_ERR_ALIGNMENT,
                "out must be 8-byte aligned");
    if (n == 0) return TSG_OK;
    hipLaunchKernelGGL(gen_bytes_kernel, dim3(grid_for((n + 7) / 8)), dim3(256), 0,
                       as_stream(stream), seed, out, n);
    return check_launch("gen_bytes");
}

extern "C" tsg_status tsg_gen_bf16_normal(tsg_stream stream, uint64_t seed, uint16_t* out,
                                          uint64_t n, float sigma, int abs_value,
                                          float divisor) {
    TSG_REQUIRE(out || n == 0, TSG_ERR_INVALID_ARGUMENT, "out is NULL");
    TSG_REQUIRE(divisor != 0.0f, TSG_ERR_INVALID_ARGUMENT, "divisor is zero");
    if (n == 0) return TSG_OK;
    hipLaunchKernelGGL(gen_bf16_normal_kernel, dim3(grid_for(n)), dim3(256), 0,
                       as_stream(stream), seed, out, n, sigma, abs_value, divisor);
    return check_launch("gen_bf16_normal");
}

extern "C" tsg_status tsg_gen_f16_normal(tsg_stream stream, uint64_t seed, uint16_t* out,
                                         uint64_t n, float sigma) {
    TSG_REQUIRE(out || n == 0, TSG_ERR_INVALID_ARGUMENT, "out is NULL");
    if (n == 0) return TSG_OK;
    hipLaunchKernelGGL(gen_f16_normal_kernel, dim3(grid_for(n)), dim3(256), 0,
                       as_stream(stream), seed, out, n, sigma);
    return check_launch("gen_f16_normal");
}
