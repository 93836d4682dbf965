// HBM read-ceiling probe for the benchmark (not part of the decode path's ABI).
//
// Streams `bytes` of a device buffer once with 16-byte loads, eight in flight
// per lane, and folds them into one word per lane so no load is dead.  Timed
// by the caller on `stream`; with the buffer far larger than the 256 MB
// Infinity Cache and a flush between runs, the rate is the achievable cold
// read bandwidth that the decode kernels' weight streams are measured against
// (the role of recipe-lna/lna2/cold_read_bw.cu:23-153 on the reference's card).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int PROBE_THREADS = 256;
constexpr int PROBE_UNROLL = 8;

__global__ __launch_bounds__(PROBE_THREADS) void probe_read_kernel(const u32x4_t* __restrict__ buf, int64_t nvec,
                                                                   uint32_t* __restrict__ sink) {
    const int64_t tid = (int64_t)blockIdx.x * PROBE_THREADS + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * PROBE_THREADS;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    int64_t i = tid;
    // whole rounds of PROBE_UNROLL loads per lane, every address in range
    for (; i + (PROBE_UNROLL - 1) * stride < nvec; i += PROBE_UNROLL * stride) {
        u32x4_t v[PROBE_UNROLL];
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) v[u] = __builtin_nontemporal_load(buf + i + u * stride);
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u];
    }
    for (; i < nvec; i += stride) acc ^= buf[i];
    sink[tid] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

extern "C" {

// Launches the probe over bytes (a multiple of 16) at buf; sink holds one
// uint32 per launched thread: blocks * 256.  Returns 0, or -1 on a bad
// argument or launch error.
int exl3_probe_read(const void* buf, int64_t bytes, uint32_t* sink, int blocks, void* stream) {
    if (!buf || !sink || bytes <= 0 || bytes % 16 || blocks < 1) return -1;
    hipLaunchKernelGGL(probe_read_kernel, dim3(blocks), dim3(PROBE_THREADS), 0, reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const u32x4_t*>(buf), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int exl3_probe_threads(void) { return PROBE_THREADS; }

}  // extern "C"
