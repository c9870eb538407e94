// stream_floor: the shortest time this GPU takes to read N bytes from HBM in one launch, the
// practical ceiling of a bandwidth-bound kernel of that size (the decode GEMV reads
// 33,216,000 bytes per launch). A bare streaming kernel - 16-byte non-temporal buffer loads,
// all of a lane's loads issued at once, one word written only if their XOR hits a magic value
// - reads distinct device copies in rotation (their total past the 256 MB Infinity Cache, so
// every launch reads HBM), for a few launch shapes; HIP events over back-to-back launches.
//
//   stream_floor [bytes] [launches]   ->  one JSON line on stdout
//
// A measurement helper of bench.py (--read-floor), not part of the library.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <cstdlib>
#include <vector>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int N>
__global__ void stream_kernel(const uint8_t* base, uint32_t bytes, uint32_t* sink) {
    // Offsets past `bytes` lie outside the buffer resource and read zeros.
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                          0x00020000);
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t nthreads = gridDim.x * blockDim.x;
    u32x4 v[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (tid + i * nthreads) * 16u, 0, 2));
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9E3779B9u) sink[tid] = acc;
}

struct Shape {
    const char* name;
    int threads;
    int per_lane;
};

void launch(const Shape& sh, const uint8_t* b, uint32_t bytes, uint32_t* sink, hipStream_t s) {
    const uint32_t chunks = (bytes + 15u) / 16u;
    const uint32_t per = static_cast<uint32_t>(sh.threads * sh.per_lane);
    const dim3 grid((chunks + per - 1u) / per);
    switch (sh.per_lane) {
        case 4: hipLaunchKernelGGL(stream_kernel<4>, grid, dim3(sh.threads), 0, s, b, bytes, sink); break;
        case 8: hipLaunchKernelGGL(stream_kernel<8>, grid, dim3(sh.threads), 0, s, b, bytes, sink); break;
        default: hipLaunchKernelGGL(stream_kernel<16>, grid, dim3(sh.threads), 0, s, b, bytes, sink); break;
    }
}

int fail(const char* what, hipError_t e) {
    std::fprintf(stderr, "stream_floor: %s: %s\n", what, hipGetErrorString(e));
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    const uint32_t bytes = argc > 1 ? static_cast<uint32_t>(std::strtoul(argv[1], nullptr, 10)) : 33216000u;
    const int launches = argc > 2 ? std::atoi(argv[2]) : 200;
    if (bytes < 16u || bytes > (1u << 30) || launches < 1) {
        std::fprintf(stderr, "stream_floor: bytes in [16, 2^30], launches >= 1\n");
        return 2;
    }
    const size_t mall = size_t{256} << 20;
    const int copies = static_cast<int>(std::max<size_t>(4, (2 * mall) / bytes + 2));
    std::vector<uint8_t*> bufs(copies, nullptr);
    hipError_t e;
    for (auto& p : bufs) {
        if ((e = hipMalloc(&p, bytes)) != hipSuccess) return fail("hipMalloc", e);
        if ((e = hipMemset(p, 1, bytes)) != hipSuccess) return fail("hipMemset", e);
    }
    uint32_t* sink = nullptr;
    const Shape shapes[] = {{"512 threads x 8 loads", 512, 8}, {"256 threads x 16 loads", 256, 16},
                            {"1024 threads x 4 loads", 1024, 4}, {"256 threads x 8 loads", 256, 8}};
    size_t max_threads = 0;
    for (const Shape& sh : shapes) {
        const size_t per = static_cast<size_t>(sh.threads) * sh.per_lane;
        max_threads = std::max(max_threads, ((bytes + 15u) / 16u + per - 1u) / per * sh.threads);
    }
    if ((e = hipMalloc(&sink, max_threads * sizeof(uint32_t))) != hipSuccess) return fail("hipMalloc", e);
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((e = hipStreamCreate(&s)) != hipSuccess) return fail("hipStreamCreate", e);
    if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess)
        return fail("hipEventCreate", e);
    double best = 1e30;
    const char* best_name = "";
    std::fprintf(stderr, "stream_floor: %u bytes, %d copies, %d launches per shape\n", bytes, copies, launches);
    for (const Shape& sh : shapes) {
        for (int i = 0; i < copies; ++i) launch(sh, bufs[i], bytes, sink, s);   // every copy read once
        if ((e = hipEventRecord(e0, s)) != hipSuccess) return fail("hipEventRecord", e);
        for (int i = 0; i < launches; ++i) launch(sh, bufs[i % copies], bytes, sink, s);
        if ((e = hipEventRecord(e1, s)) != hipSuccess) return fail("hipEventRecord", e);
        if ((e = hipEventSynchronize(e1)) != hipSuccess) return fail("hipEventSynchronize", e);
        if ((e = hipGetLastError()) != hipSuccess) return fail("launch", e);
        float ms = 0.0f;
        if ((e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess) return fail("hipEventElapsedTime", e);
        const double us = 1e3 * ms / launches;
        std::fprintf(stderr, "stream_floor: %-24s %7.2f us  %6.0f GB/s\n", sh.name, us, bytes / us / 1e3);
        if (us < best) {
            best = us;
            best_name = sh.name;
        }
    }
    std::printf("{\"bytes\": %u, \"us\": %.3f, \"gbs\": %.1f, \"shape\": \"%s\", \"copies\": %d, \"launches\": %d}\n",
                bytes, best, bytes / best / 1e3, best_name, copies, launches);
    (void)hipStreamDestroy(s);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    for (auto* p : bufs) (void)hipFree(p);
    (void)hipFree(sink);
    return 0;
}
