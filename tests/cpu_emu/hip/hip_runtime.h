// hip/hip_runtime.h for the CPU emulation build (TEST INFRASTRUCTURE ONLY).
//
// Lets the unmodified kernel source (gpu-forge_amd/csrc/radix_kernels.hip) and
// host runtime (gpu-forge_amd/csrc/forge_sort.cpp) compile as ordinary C++ and
// run on the CPU under tests/cpu_emu/hip_emu.cpp: every GPU thread is a fiber,
// every block runs on its own OS thread (blocks run concurrently, so the
// decoupled look-back really races), wave64 intrinsics are lane rendezvous,
// and device buffers sit against PROT_NONE guard pages so an out-of-bounds
// access faults on the CPU.  Nothing here is linked into the product.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __constant__
#define __shared__ static thread_local
#define __align__(n) __attribute__((aligned(n)))

struct uint4 { uint32_t x, y, z, w; };
struct emu_dim3 { uint32_t x, y, z; };

namespace emu {
emu_dim3 thread_idx();
emu_dim3 block_idx();
emu_dim3 block_dim();
emu_dim3 grid_dim();
void syncthreads();
int syncthreads_or(int pred);
// wave64 operations over the lanes of the calling thread's wave that reach them
uint64_t ballot(int pred);
int all(int pred);
uint32_t shfl_up(uint32_t v, unsigned off);
uint32_t readfirstlane(uint32_t v);
uint32_t readlane(uint32_t v, uint32_t src);
void sleep_hint();
void wave_barrier();
unsigned lane();
}  // namespace emu

#define threadIdx (::emu::thread_idx())
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())

inline void __syncthreads() { emu::syncthreads(); }
inline int __syncthreads_or(int p) { return emu::syncthreads_or(p); }
inline void __threadfence() { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
// every emulated memory operation has completed when the lane continues
#define __builtin_amdgcn_s_waitcnt(imm) __atomic_thread_fence(__ATOMIC_SEQ_CST)
inline unsigned long long __ballot(int p) { return emu::ballot(p); }
inline int __all(int p) { return emu::all(p); }
inline uint32_t __shfl_up(uint32_t v, unsigned off, int /*width*/) { return emu::shfl_up(v, off); }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }

// ---- AMDGPU builtins used by the kernels ----------------------------------
inline uint32_t emu_readfirstlane(uint32_t v) { return emu::readfirstlane(v); }
inline uint64_t emu_uicmp(uint32_t a, uint32_t b, int pred) {
    bool r;
    switch (pred) {
        case 32: r = a == b; break;   // ICMP_EQ
        case 33: r = a != b; break;   // ICMP_NE
        case 34: r = a > b; break;    // ICMP_UGT
        case 35: r = a >= b; break;
        case 36: r = a < b; break;
        case 37: r = a <= b; break;
        default: r = false; break;
    }
    return emu::ballot(r);
}
inline int32_t emu_sbfe(int32_t x, int off, int width) {
    if (width == 0) return 0;
    uint32_t u = ((uint32_t)x >> off) & ((width >= 32) ? 0xFFFFFFFFu : ((1u << width) - 1u));
    if (width < 32 && (u >> (width - 1)) & 1u) u |= ~((1u << width) - 1u);
    return (int32_t)u;
}
// v_bfe_u32: offset and width are taken from their low 5 bits.
inline uint32_t emu_ubfe(uint32_t x, uint32_t off, uint32_t width) {
    off &= 31u; width &= 31u;
    if (width == 0) return 0u;
    return (x >> off) & ((1u << width) - 1u);
}
// v_perm_b32: result byte i is chosen by selector byte i from the bytes of
// {src0, src1} (0-3: src1, 4-7: src0), 8-11 sign bits, 12 = 0x00, >= 13 = 0xFF.
inline uint32_t emu_perm(uint32_t src0, uint32_t src1, uint32_t sel) {
    const uint64_t v = ((uint64_t)src0 << 32) | src1;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t s = (sel >> (8 * i)) & 0xFFu;
        uint32_t b;
        if (s < 8u) b = (uint32_t)(v >> (8 * s)) & 0xFFu;
        else if (s < 12u) b = ((v >> (16 * (s - 8u) + 15)) & 1u) ? 0xFFu : 0x00u;
        else if (s == 12u) b = 0x00u;
        else b = 0xFFu;
        r |= b << (8 * i);
    }
    return r;
}
inline uint32_t emu_bitop3(uint32_t a, uint32_t b, uint32_t c, uint32_t tt) {
    uint32_t r = 0;
    for (int i = 0; i < 8; ++i) {
        if (!((tt >> i) & 1u)) continue;
        const uint32_t ma = (i & 4) ? a : ~a, mb = (i & 2) ? b : ~b, mc = (i & 1) ? c : ~c;
        r |= ma & mb & mc;
    }
    return r;
}
inline uint32_t emu_mbcnt_lo(uint32_t mask, uint32_t acc) {
    const unsigned l = emu::lane();
    const uint32_t below = l >= 32 ? 0xFFFFFFFFu : ((1u << l) - 1u);
    return acc + (uint32_t)__builtin_popcount(mask & below);
}
inline uint32_t emu_mbcnt_hi(uint32_t mask, uint32_t acc) {
    const unsigned l = emu::lane();
    const uint32_t below = l < 32 ? 0u : ((l - 32) >= 32 ? 0xFFFFFFFFu : ((1u << (l - 32)) - 1u));
    return acc + (uint32_t)__builtin_popcount(mask & below);
}
#define __builtin_amdgcn_readfirstlane(v) emu_readfirstlane((uint32_t)(v))
#define __builtin_amdgcn_readlane(v, l) ::emu::readlane((uint32_t)(v), (uint32_t)(l))
#define __builtin_amdgcn_uicmp(a, b, p) emu_uicmp((uint32_t)(a), (uint32_t)(b), (p))
#define __builtin_amdgcn_sbfe(x, o, w) emu_sbfe((int32_t)(x), (o), (w))
#define __builtin_amdgcn_ubfe(x, o, w) emu_ubfe((uint32_t)(x), (o), (w))
#define __builtin_amdgcn_perm(a, b, s) emu_perm((uint32_t)(a), (uint32_t)(b), (uint32_t)(s))
#define __builtin_amdgcn_bitop3_b32(a, b, c, t) emu_bitop3((a), (b), (c), (t))
#define __builtin_amdgcn_mbcnt_lo(m, a) emu_mbcnt_lo((m), (a))
#define __builtin_amdgcn_mbcnt_hi(m, a) emu_mbcnt_hi((m), (a))
#define __builtin_amdgcn_s_sleep(n) emu::sleep_hint()
#define __builtin_amdgcn_wave_barrier() emu::wave_barrier()

// ---- atomics ------------------------------------------------------------------
#define __HIP_MEMORY_SCOPE_WORKGROUP 2
#define __HIP_MEMORY_SCOPE_AGENT 3
#define __HIP_MEMORY_SCOPE_SYSTEM 4
#define __hip_atomic_load(p, order, scope) __atomic_load_n((p), __ATOMIC_ACQUIRE)
#define __hip_atomic_store(p, v, order, scope) __atomic_store_n((p), (v), __ATOMIC_RELEASE)
#define __hip_atomic_fetch_or(p, v, order, scope) __atomic_fetch_or((p), (v), __ATOMIC_ACQ_REL)
#define __hip_atomic_fetch_add(p, v, order, scope) __atomic_fetch_add((p), (v), __ATOMIC_ACQ_REL)
// HIP's device min/max for integers
template <class T> inline T min(T a, T b) { return b < a ? b : a; }
template <class T> inline T max(T a, T b) { return a < b ? b : a; }
inline uint32_t atomicAdd(uint32_t* p, uint32_t v) { return __atomic_fetch_add(p, v, __ATOMIC_ACQ_REL); }
inline unsigned long long atomicAdd(unsigned long long* p, unsigned long long v) {
    return __atomic_fetch_add(p, v, __ATOMIC_ACQ_REL);
}
inline uint32_t atomicOr(uint32_t* p, uint32_t v) { return __atomic_fetch_or(p, v, __ATOMIC_ACQ_REL); }
inline uint32_t atomicMax(uint32_t* p, uint32_t v) {
    uint32_t old = __atomic_load_n(p, __ATOMIC_ACQUIRE);
    while (old < v && !__atomic_compare_exchange_n(p, &old, v, false, __ATOMIC_ACQ_REL, __ATOMIC_ACQUIRE)) {
    }
    return old;
}
inline unsigned long long atomicOr(unsigned long long* p, unsigned long long v) {
    return __atomic_fetch_or(p, v, __ATOMIC_ACQ_REL);
}

// ---- host runtime API (the subset forge_sort.cpp uses) -------------------------
typedef int hipError_t;
#define hipSuccess 0
#define hipErrorInvalidValue 1
#define hipErrorOutOfMemory 2
#define hipErrorNotFound 500
typedef struct emu_stream* hipStream_t;
typedef struct emu_event* hipEvent_t;
typedef struct emu_module* hipModule_t;
typedef struct emu_function* hipFunction_t;
typedef void* hipDeviceptr_t;
typedef enum { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2,
               hipMemcpyDeviceToDevice = 3, hipMemcpyDefault = 4 } hipMemcpyKind;
typedef enum { hipDeviceAttributeMultiprocessorCount = 1 } hipDeviceAttribute_t;
#define hipStreamNonBlocking 1
#define hipHostMallocDefault 0

hipError_t hipGetDeviceCount(int*);
hipError_t hipSetDevice(int);
hipError_t hipDeviceGetAttribute(int*, hipDeviceAttribute_t, int);
hipError_t hipGetLastError(void);
const char* hipGetErrorString(hipError_t);
hipError_t hipStreamCreateWithFlags(hipStream_t*, unsigned);
typedef enum { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1,
               hipStreamCaptureStatusInvalidated = 2 } hipStreamCaptureStatus;
hipError_t hipStreamBeginCapture(hipStream_t, int);
hipError_t hipStreamEndCapture(hipStream_t, void**);
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus*);
hipError_t hipStreamDestroy(hipStream_t);
hipError_t hipStreamSynchronize(hipStream_t);
hipError_t hipDeviceSynchronize(void);
hipError_t hipMalloc(void**, size_t);
template <typename T> inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc((void**)p, n); }
hipError_t hipFree(void*);
hipError_t hipHostMalloc(void**, size_t, unsigned);
template <typename T> inline hipError_t hipHostMalloc(T** p, size_t n, unsigned f) { return hipHostMalloc((void**)p, n, f); }
hipError_t hipHostFree(void*);
hipError_t hipMemset(void*, int, size_t);
hipError_t hipMemcpy(void*, const void*, size_t, hipMemcpyKind);
hipError_t hipMemcpyAsync(void*, const void*, size_t, hipMemcpyKind, hipStream_t);
hipError_t hipMemcpyDtoH(void*, hipDeviceptr_t, size_t);
hipError_t hipModuleLoad(hipModule_t*, const char*);
hipError_t hipModuleUnload(hipModule_t);
hipError_t hipModuleGetFunction(hipFunction_t*, hipModule_t, const char*);
hipError_t hipModuleGetGlobal(hipDeviceptr_t*, size_t*, hipModule_t, const char*);
hipError_t hipModuleLaunchKernel(hipFunction_t, unsigned, unsigned, unsigned, unsigned, unsigned, unsigned,
                                 unsigned, hipStream_t, void**, void**);
hipError_t hipEventCreate(hipEvent_t*);
hipError_t hipEventDestroy(hipEvent_t);
hipError_t hipEventRecord(hipEvent_t, hipStream_t);
hipError_t hipEventSynchronize(hipEvent_t);
hipError_t hipEventElapsedTime(float*, hipEvent_t, hipEvent_t);
