// CPU stand-in for the HIP API that decode_step.hip and cw_internal.hpp use,
// for a CPU execution of the fused decode-step kernel (step_emu.cpp).  Test
// infrastructure only: nothing in the library is built with it.
//
// Every thread of the grid runs the kernel as a fiber; the wave-level
// operations (shuffles, DPP moves) and the workgroup barrier are collectives
// over the wave's 64 / the workgroup's fibers, atomics are plain memory
// operations (the fibers of one OS thread never interleave inside one), and
// buffer loads apply the hardware's range check (out-of-range reads give
// zeros).  Global memory is host memory, so an access outside an allocation
// is reported by AddressSanitizer; each workgroup's LDS is a host buffer of
// exactly the bytes the launch provides.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#define CW_STEP_HOOKS 1

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)

// ---------------------------------------------------------------- host API stubs

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorNotSupported = 801 };
typedef struct emu_stream *hipStream_t;
typedef struct emu_event *hipEvent_t;
enum { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };

struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};

inline const char *hipGetErrorString(hipError_t) { return "not available in the CPU execution"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipFuncSetAttribute(const void *, int, int) { return hipErrorNotSupported; }
template <class F>
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int *n, F, int, size_t) {
    *n = 0;
    return hipErrorNotSupported;
}
inline hipError_t hipLaunchCooperativeKernel(const void *, dim3, dim3, void **, unsigned,
                                             hipStream_t) {
    return hipErrorNotSupported;
}
template <class... A>
inline void hipLaunchKernelGGL(A...) {}
template <class... A>
inline void hipExtLaunchKernelGGL(A...) {}

// ---------------------------------------------------------------- device side

struct float4 {
    float x, y, z, w;
};
struct uint4 {
    uint32_t x, y, z, w;
};
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline uint4 make_uint4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) { return uint4{x, y, z, w}; }

// a buffer resource: base and size in bytes (the range check)
struct emu_rsrc {
    const unsigned char *base;
    uint32_t bytes;
};
typedef emu_rsrc __amdgpu_buffer_rsrc_t;

namespace emu {

struct Fiber;
Fiber *cur();
void yield();
void progress();
uint32_t wave_op(uint32_t v, int kind, int param);  // kinds below
void sync_threads();
unsigned long long clock();
enum { OP_SHFL = 1, OP_SHFL_XOR = 2, OP_DPP = 3, OP_FIRST = 4 };

struct Idx {
    unsigned x, y, z;
};
const Idx &thread_idx();
const Idx &block_idx();
const Idx &block_dim();
const Idx &grid_dim();
void *wg_static(size_t bytes);
void *wg_dynamic();

template <class T>
inline uint32_t bits(T v) {
    static_assert(sizeof(T) == 4, "32-bit lane values");
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}
template <class T>
inline T from_bits(uint32_t u) {
    T v;
    memcpy(&v, &u, 4);
    return v;
}

template <unsigned N>
inline void rsrc_load(const emu_rsrc &r, int voff, int soff, void *out) {
    const long off = (long)voff + (long)soff;
    if (off < 0 || (unsigned long)off + N > r.bytes) {  // out of range: zeros
        memset(out, 0, N);
        return;
    }
    memcpy(out, r.base + off, N);
}

}  // namespace emu

#define threadIdx (::emu::thread_idx())
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())

#define CW_OPAQUE_S(v) ((void)0)
#define CW_OPAQUE_V(v) ((void)0)
#define CW_WG_SHARED(T, name) T &name = *static_cast<T *>(::emu::wg_static(sizeof(T)))
#define CW_WG_DYNAMIC(T, name) T *name = static_cast<T *>(::emu::wg_dynamic())

inline void __syncthreads() { emu::sync_threads(); }
template <class T>
inline T __shfl_xor(T v, int mask, int = 64) {
    return emu::from_bits<T>(emu::wave_op(emu::bits(v), emu::OP_SHFL_XOR, mask));
}
template <class T>
inline T __shfl(T v, int src, int = 64) {
    return emu::from_bits<T>(emu::wave_op(emu::bits(v), emu::OP_SHFL, src));
}
inline unsigned long long wall_clock64() { return emu::clock(); }

#define __builtin_amdgcn_s_waitcnt(x) ((void)0)
#define __builtin_amdgcn_sched_barrier(x) ((void)0)
// lane 0's value; the kernel applies it to values it holds uniform over the
// wave, which the collective checks (a lane holding another value aborts)
template <class T>
inline T emu_readfirstlane(T v) {
    return emu::from_bits<T>(emu::wave_op(emu::bits(v), emu::OP_FIRST, 0));
}
#define __builtin_amdgcn_readfirstlane(x) emu_readfirstlane(x)
#define __builtin_amdgcn_mov_dpp(v, ctrl, rm, bm, bc) \
    ((int)::emu::wave_op((uint32_t)(v), ::emu::OP_DPP, (ctrl)))
inline emu_rsrc emu_make_rsrc(const void *p, int, uint32_t bytes, int) {
    return emu_rsrc{static_cast<const unsigned char *>(p), bytes};
}
#define __builtin_amdgcn_make_buffer_rsrc(p, stride, n, flags) emu_make_rsrc((p), (stride), (n), (flags))
struct emu_u128 {
    uint32_t v[4];
};
inline emu_u128 __builtin_amdgcn_raw_buffer_load_b128(emu_rsrc r, int voff, int soff, int) {
    emu_u128 o;
    emu::rsrc_load<16>(r, voff, soff, o.v);
    return o;
}
inline uint32_t __builtin_amdgcn_raw_buffer_load_b32(emu_rsrc r, int voff, int soff, int) {
    uint32_t o;
    emu::rsrc_load<4>(r, voff, soff, &o);
    return o;
}
inline unsigned short __builtin_amdgcn_raw_buffer_load_b16(emu_rsrc r, int voff, int soff, int) {
    unsigned short o;
    emu::rsrc_load<2>(r, voff, soff, &o);
    return o;
}

#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
template <class T>
inline T emu_atomic_load(const T *p) {
    const T v = *p;
    emu::yield();  // a polling loop lets the other fibers run
    return v;
}
template <class T, class V>
inline void emu_atomic_store(T *p, V v) {
    *p = (T)v;
    emu::progress();
}
template <class T, class V>
inline T emu_atomic_add(T *p, V v) {
    const T old = *p;
    *p = (T)(old + (T)v);
    emu::progress();
    return old;
}
#define __hip_atomic_load(p, order, scope) emu_atomic_load(p)
#define __hip_atomic_store(p, v, order, scope) emu_atomic_store((p), (v))
#define __hip_atomic_fetch_add(p, v, order, scope) emu_atomic_add((p), (v))
