// CPU emulation shim for <hip/hip_runtime.h> (test infrastructure only).
//
// Lets the sampler's kernel sources (vllm_mps_amd/csrc) compile as host C++
// so that tests/emu/emu.cpp can run every workgroup on the CPU: each lane is
// a cooperative fiber, __syncthreads() waits for every live lane of the
// block, and the wave64 intrinsics (__shfl*, __ballot, readfirstlane) wait
// for every live lane of the wave and then exchange values exactly as the
// hardware does.  Under AddressSanitizer and -fsanitize=bounds the run then
// checks every global and LDS access the kernels make.
#pragma once

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <functional>
#include <type_traits>

#define __global__
#define __device__
#define __align__(n) __attribute__((aligned(n)))
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

namespace emu {

// ---------------------------------------------------------------- lanes and blocks
const dim3 &thread_idx();
const dim3 &block_idx();
const dim3 &block_dim();
const dim3 &grid_dim();

void syncthreads(const char *site);
// wave ops on 64-bit payloads; kind selects the exchange
enum WaveOp : int { OP_SHFL = 0, OP_XOR = 1, OP_UP = 2, OP_DOWN = 3, OP_BALLOT = 4, OP_FIRST = 5 };
uint64_t wave_op(int kind, uint64_t v, int arg, int width, const char *site);

void launch(dim3 grid, dim3 block, const std::function<void()> &fn, const char *name);

template <class T> inline uint64_t to_u64(T v)
{
    static_assert(sizeof(T) <= 8, "payload up to 8 bytes");
    uint64_t u = 0;
    memcpy(&u, &v, sizeof(T));
    return u;
}
template <class T> inline T from_u64(uint64_t u)
{
    T v;
    memcpy(&v, &u, sizeof(T));
    return v;
}

}  // namespace emu

#define EMU_STR2(x) #x
#define EMU_STR(x) EMU_STR2(x)
#define EMU_SITE __FILE__ ":" EMU_STR(__LINE__)

#define threadIdx (emu::thread_idx())
#define blockIdx (emu::block_idx())
#define blockDim (emu::block_dim())
#define gridDim (emu::grid_dim())

#define __syncthreads() emu::syncthreads(EMU_SITE)

template <class T> inline T emu_shfl(T v, int src, int width, const char *site)
{ return emu::from_u64<T>(emu::wave_op(emu::OP_SHFL, emu::to_u64(v), src, width, site)); }
template <class T> inline T emu_shfl_xor(T v, int m, int width, const char *site)
{ return emu::from_u64<T>(emu::wave_op(emu::OP_XOR, emu::to_u64(v), m, width, site)); }
template <class T> inline T emu_shfl_up(T v, int d, int width, const char *site)
{ return emu::from_u64<T>(emu::wave_op(emu::OP_UP, emu::to_u64(v), d, width, site)); }
template <class T> inline T emu_shfl_down(T v, int d, int width, const char *site)
{ return emu::from_u64<T>(emu::wave_op(emu::OP_DOWN, emu::to_u64(v), d, width, site)); }
template <class T> inline T emu_first(T v, const char *site)
{ return emu::from_u64<T>(emu::wave_op(emu::OP_FIRST, emu::to_u64(v), 0, 64, site)); }

#define EMU_W(w, ...) w
#define __shfl(v, s, ...) emu_shfl((v), (s), EMU_W(__VA_ARGS__ __VA_OPT__(,) 64), EMU_SITE)
#define __shfl_xor(v, m, ...) emu_shfl_xor((v), (m), EMU_W(__VA_ARGS__ __VA_OPT__(,) 64), EMU_SITE)
#define __shfl_up(v, d, ...) emu_shfl_up((v), (d), EMU_W(__VA_ARGS__ __VA_OPT__(,) 64), EMU_SITE)
#define __shfl_down(v, d, ...) emu_shfl_down((v), (d), EMU_W(__VA_ARGS__ __VA_OPT__(,) 64), EMU_SITE)
#define __ballot(p) emu::wave_op(emu::OP_BALLOT, (uint64_t)((p) ? 1 : 0), 0, 64, EMU_SITE)
#define __builtin_amdgcn_readfirstlane(v) emu_first((v), EMU_SITE)
#define __builtin_amdgcn_exp2f(f) exp2f(f)
// phase timestamps of a MIS_TRACE build: a global counter stands in for the
// real-time clock, a plain store for the device-scope store
namespace emu { uint64_t clock_tick(); }
#define __builtin_amdgcn_s_memrealtime() emu::clock_tick()
#define __hip_atomic_store(p, v, order, scope) (*(p) = (v))

// HIP's device integer min / max
template <class T> inline T min(T a, T b) { return b < a ? b : a; }
template <class T> inline T max(T a, T b) { return a < b ? b : a; }

inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __popc(unsigned v) { return __builtin_popcount(v); }

// Lanes run one at a time, so atomics are plain read-modify-writes.
template <class T, class U> inline T atomicAdd(T *p, U v) { T o = *p; *p = (T)(o + (T)v); return o; }
// workgroups run one after another here: device-scope fences have nothing to order
#define __threadfence() ((void)0)
template <class T, class U> inline T atomicMin(T *p, U v) { T o = *p; if ((T)v < o) *p = (T)v; return o; }
template <class T, class U> inline T atomicMax(T *p, U v) { T o = *p; if ((T)v > o) *p = (T)v; return o; }
template <class T, class U> inline T atomicOr(T *p, U v) { T o = *p; *p = (T)(o | (T)v); return o; }
template <class T, class U> inline T atomicExch(T *p, U v) { T o = *p; *p = (T)v; return o; }

// ---------------------------------------------------------------- host API
typedef int hipError_t;
enum : int { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorInvalidDevice = 101 };
typedef struct emu_stream *hipStream_t;
typedef struct emu_event *hipEvent_t;
enum : unsigned { hipStreamNonBlocking = 1u, hipEventDisableTiming = 2u };

inline hipError_t hipGetDevice(int *d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetLastError() { return hipSuccess; }
// a __device__ variable is an ordinary host object here: its address is the symbol's
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void **p, const void *sym) { *p = const_cast<void *>(sym); return hipSuccess; }
inline hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) { *s = (hipStream_t)(uintptr_t)0x5151; return hipSuccess; }
inline hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) { *e = (hipEvent_t)(uintptr_t)0xe7e7; return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }
inline hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
inline hipError_t hipMemsetAsync(void *p, int v, size_t n, hipStream_t) { memset(p, v, n); return hipSuccess; }

// Kernels run to completion in launch order (one stream in effect).
#define hipLaunchKernelGGL(k, grid, block, shmem, stream, ...) \
    emu::launch(dim3(grid), dim3(block), [&]() { k(__VA_ARGS__); }, #k)
