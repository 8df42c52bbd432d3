// hipCUB DeviceRadixSort on device buffers, as an independent yardstick for
// the forge-sort HIP path (TEST INFRASTRUCTURE ONLY: loaded by
// tests/test_gpu_parity.py, never linked into the product).  hipCUB comes
// from the ROCm headers (rocPRIM's onesweep radix sort underneath).
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <stdint.h>

namespace {

template <typename K>
int sort_keys(const K* d_in, K* d_out, uint64_t n, float* ms) {
    size_t temp_bytes = 0;
    if (hipcub::DeviceRadixSort::SortKeys(nullptr, temp_bytes, d_in, d_out, (int)n) != hipSuccess) return 1;
    void* temp = nullptr;
    if (hipMalloc(&temp, temp_bytes ? temp_bytes : 1) != hipSuccess) return 2;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    (void)hipEventRecord(a, 0);
    hipError_t e = hipcub::DeviceRadixSort::SortKeys(temp, temp_bytes, d_in, d_out, (int)n);
    (void)hipEventRecord(b, 0);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (ms) (void)hipEventElapsedTime(ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(temp);
    return e == hipSuccess ? 0 : 3;
}

template <typename K>
int sort_pairs(const K* k_in, K* k_out, const uint32_t* v_in, uint32_t* v_out, uint64_t n, float* ms) {
    size_t temp_bytes = 0;
    if (hipcub::DeviceRadixSort::SortPairs(nullptr, temp_bytes, k_in, k_out, v_in, v_out, (int)n) != hipSuccess)
        return 1;
    void* temp = nullptr;
    if (hipMalloc(&temp, temp_bytes ? temp_bytes : 1) != hipSuccess) return 2;
    hipEvent_t a, b;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    (void)hipEventRecord(a, 0);
    hipError_t e = hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, k_in, k_out, v_in, v_out, (int)n);
    (void)hipEventRecord(b, 0);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    if (ms) (void)hipEventElapsedTime(ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(temp);
    return e == hipSuccess ? 0 : 3;
}

}  // namespace

extern "C" {
// Unsigned keys (the caller applies any order-preserving transform).  n < 2^31.
int xc_sort_keys_u32(const uint32_t* d_in, uint32_t* d_out, uint64_t n, float* ms) {
    return sort_keys(d_in, d_out, n, ms);
}
int xc_sort_keys_u64(const uint64_t* d_in, uint64_t* d_out, uint64_t n, float* ms) {
    return sort_keys(d_in, d_out, n, ms);
}
int xc_sort_pairs_u32(const uint32_t* k_in, uint32_t* k_out, const uint32_t* v_in, uint32_t* v_out, uint64_t n,
                      float* ms) {
    return sort_pairs(k_in, k_out, v_in, v_out, n, ms);
}
}
