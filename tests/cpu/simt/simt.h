/*
 * simt.h — a CPU emulator of the HIP execution model, for debugging and testing the library's kernels
 * on the host (test infrastructure; the product never links it).
 *
 * Every GPU thread of a workgroup is a fiber (ucontext); workgroups run one after another. Wave
 * operations (__shfl*, __ballot) rendezvous the 64 fibers of a wavefront, __syncthreads() all fibers
 * of the workgroup; `__shared__` variables become function statics, shared by the fibers of the
 * running workgroup. Device memory is host memory, so AddressSanitizer sees every access. Atomics
 * are plain read-modify-writes (fibers never preempt each other inside one).
 */
#pragma once
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include <algorithm>
#include <functional>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#if defined(SIMT_POISON_LDS)
#define __shared__ __attribute__((section("simt_lds"))) static
#else
#define __shared__ static
#endif
#define __constant__

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct alignas(16) float4 {
  float x, y, z, w;
};
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }

namespace simt {
struct Block;
dim3 tidx();
dim3 bidx();
dim3 bdim();
dim3 gdim();
void sync_block_at(const char *file, int line);
void sync_wave();
void wave_site(const char *file, int line);
uint64_t *wave_slots();
int lane_id();
void launch(dim3 grid, dim3 block, const std::function<void()> &body);
}  // namespace simt

#define threadIdx (simt::tidx())
#define blockIdx (simt::bidx())
#define blockDim (simt::bdim())
#define gridDim (simt::gdim())

#define __syncthreads() simt::sync_block_at(__FILE__, __LINE__)
inline void __threadfence() {}

template <class T>
inline T simt_exchange(T v, int src) {
  static_assert(sizeof(T) <= 8, "wave exchange of a value wider than 8 bytes");
  uint64_t *slots = simt::wave_slots();
  uint64_t b = 0;
  memcpy(&b, &v, sizeof(T));
  slots[simt::lane_id()] = b;
  simt::sync_wave();
  uint64_t r = slots[src & 63];
  simt::sync_wave();
  T out;
  memcpy(&out, &r, sizeof(T));
  return out;
}
template <class T>
inline T simt_shfl(T v, int src, int width = 64) {
  (void)width;
  return simt_exchange(v, src);
}
template <class T>
inline T simt_shfl_up(T v, unsigned k, int width = 64) {
  (void)width;
  int l = simt::lane_id();
  return simt_exchange(v, l >= (int)k ? l - (int)k : l);
}
template <class T>
inline T simt_shfl_down(T v, unsigned k, int width = 64) {
  (void)width;
  int l = simt::lane_id();
  return simt_exchange(v, l + (int)k < 64 ? l + (int)k : l);
}
template <class T>
inline T simt_shfl_xor(T v, int k, int width = 64) {
  (void)width;
  return simt_exchange(v, simt::lane_id() ^ k);
}
inline unsigned long long simt_ballot(int pred) {
  uint64_t *slots = simt::wave_slots();
  slots[simt::lane_id()] = pred ? 1u : 0u;
  simt::sync_wave();
  unsigned long long m = 0;
  for (int i = 0; i < 64; i++)
    if (slots[i]) m |= 1ull << i;
  simt::sync_wave();
  return m;
}
/* gfx9 DPP move: row_shr:1..15 (0x111..0x11f), row_bcast:15 (0x142), row_bcast:31 (0x143); lanes whose
 * row (lane/16) is off in row_mask or bank ((lane%16)/4) off in bank_mask keep `old`; an enabled lane
 * whose source is out of range reads 0 with bound_ctrl, else keeps `old` */
inline int simt_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  uint64_t *slots = simt::wave_slots();
  const int lane = simt::lane_id();
  slots[lane] = (uint32_t)src;
  simt::sync_wave();
  int out = old;
  const int row = lane >> 4, bank = (lane & 15) >> 2;
  if (((row_mask >> row) & 1) && ((bank_mask >> bank) & 1)) {
    int srcl = -1;
    if (ctrl >= 0x111 && ctrl <= 0x11f) {
      const int k = ctrl - 0x110;
      if ((lane & 15) >= k) srcl = lane - k;
    } else if (ctrl == 0x142) {
      if (row >= 1) srcl = row * 16 - 1;
    } else if (ctrl == 0x143) {
      if (row >= 2) srcl = 31;
    } else {
      abort(); /* a DPP control the emulator does not model */
    }
    if (srcl >= 0) out = (int)(uint32_t)slots[srcl];
    else if (bound_ctrl) out = 0;
  }
  simt::sync_wave();
  return out;
}
inline int simt_readlane(int v, int l) {
  uint64_t *slots = simt::wave_slots();
  slots[simt::lane_id()] = (uint32_t)v;
  simt::sync_wave();
  int r = (int)(uint32_t)slots[l & 63];
  simt::sync_wave();
  return r;
}

/* every wave operation names its call site: lanes of one wave meeting at different sites (a wave
 * operation in divergent code) abort the emulation */
#define __shfl(...) (simt::wave_site(__FILE__, __LINE__), simt_shfl(__VA_ARGS__))
#define __shfl_up(...) (simt::wave_site(__FILE__, __LINE__), simt_shfl_up(__VA_ARGS__))
#define __shfl_xor(...) (simt::wave_site(__FILE__, __LINE__), simt_shfl_xor(__VA_ARGS__))
#define __shfl_down(...) (simt::wave_site(__FILE__, __LINE__), simt_shfl_down(__VA_ARGS__))
#define __ballot(...) (simt::wave_site(__FILE__, __LINE__), simt_ballot(__VA_ARGS__))
#define __builtin_amdgcn_update_dpp(...) (simt::wave_site(__FILE__, __LINE__), simt_update_dpp(__VA_ARGS__))
#define __builtin_amdgcn_readlane(...) (simt::wave_site(__FILE__, __LINE__), simt_readlane(__VA_ARGS__))

inline int __ffs(int x) { return ffs(x); }
inline int __ffs(unsigned x) { return ffs((int)x); }
inline int __ffsll(long long x) { return ffsll(x); }
inline int __ffsll(unsigned long long x) { return ffsll((long long)x); }
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
inline int __popc(unsigned x) { return __builtin_popcount(x); }
inline int __clz(int x) { return x ? __builtin_clz((unsigned)x) : 32; }
inline int __clzll(long long x) { return x ? __builtin_clzll((unsigned long long)x) : 64; }
inline uint64_t __umul64hi(uint64_t a, uint64_t b) { return (uint64_t)(((unsigned __int128)a * b) >> 64); }
inline float __expf(float x) { return expf(x); }
inline float __logf(float x) { return logf(x); }
using std::max;
using std::min;

template <class T>
inline T atomicAdd(T *p, T v) {
  T o = *p;
  *p = o + v;
  return o;
}
template <class T>
inline T atomicOr(T *p, T v) {
  T o = *p;
  *p = o | v;
  return o;
}
template <class T>
inline T atomicMin(T *p, T v) {
  T o = *p;
  *p = std::min(o, v);
  return o;
}
template <class T>
inline T atomicMax(T *p, T v) {
  T o = *p;
  *p = std::max(o, v);
  return o;
}
template <class T>
inline T atomicCAS(T *p, T cmp, T v) {
  T o = *p;
  if (o == cmp) *p = v;
  return o;
}

/* ---- runtime API subset used by the library's host code ---- */
typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1 };
typedef struct simt_stream *hipStream_t;
typedef struct simt_event *hipEvent_t;
/* graph capture has no CPU emulation: the entry points report it unsupported */
typedef struct simt_graph *hipGraph_t;
typedef struct simt_graph_exec *hipGraphExec_t;
enum { hipStreamCaptureModeThreadLocal = 1, hipErrorNotSupported = 801 };
enum hipMemcpyKind { hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice, hipMemcpyHostToHost };
#define hipStreamNonBlocking 1
inline const char *hipGetErrorString(hipError_t) { return "simt"; }
inline hipError_t hipSetDevice(int) { return hipSuccess; }
/* a __device__ variable is a host variable: its "device address" is its address */
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void **p, const void *sym) {
  *p = const_cast<void *>(sym);
  return hipSuccess;
}
inline hipError_t hipStreamBeginCapture(hipStream_t, int) { return hipErrorNotSupported; }
inline hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t *) { return hipErrorNotSupported; }
inline hipError_t hipGraphInstantiate(hipGraphExec_t *, hipGraph_t, void *, void *, size_t) { return hipErrorNotSupported; }
inline hipError_t hipGraphDestroy(hipGraph_t) { return hipErrorNotSupported; }
inline hipError_t hipGraphLaunch(hipGraphExec_t, hipStream_t) { return hipErrorNotSupported; }
inline hipError_t hipGraphExecDestroy(hipGraphExec_t) { return hipErrorNotSupported; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipMalloc(void **p, size_t n) {
  *p = malloc(n);
  if (*p) memset(*p, 0xA5, n); /* uninitialised device memory is not zero */
  return *p ? hipSuccess : hipErrorInvalidValue;
}
inline hipError_t hipFree(void *p) {
  free(p);
  return hipSuccess;
}
inline hipError_t hipHostMalloc(void **p, size_t n, unsigned = 0) { return hipMalloc(p, n); }
inline hipError_t hipHostFree(void *p) { return hipFree(p); }
inline hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) {
  memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind, hipStream_t) {
  memcpy(d, s, n);
  return hipSuccess;
}
inline hipError_t hipMemset(void *d, int v, size_t n) {
  memset(d, v, n);
  return hipSuccess;
}
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
inline hipError_t hipMemsetAsync(void *d, int v, size_t n, hipStream_t) {
  memset(d, v, n);
  return hipSuccess;
}
inline hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) {
  *s = (hipStream_t)0x1;
  return hipSuccess;
}
inline hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
enum { hipErrorNotReady = 600 };
/* a 4-CU device: grids above 20 row-pass workgroups take the library's two-half row pass, so the emulated
 * workloads exercise both instances */
enum { hipDeviceAttributeMultiprocessorCount = 63 };
inline hipError_t hipDeviceGetAttribute(int *v, int, int) { *v = 4; return hipSuccess; }
inline hipError_t hipStreamQuery(hipStream_t) { return hipSuccess; } /* launches run to completion */
inline hipError_t hipEventCreate(hipEvent_t *e) {
  *e = (hipEvent_t)0x1;
  return hipSuccess;
}
inline hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventElapsedTime(float *ms, hipEvent_t, hipEvent_t) {
  *ms = 0.0f;
  return hipSuccess;
}

#define hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ...) \
  simt::launch(dim3(grid), dim3(block), [&]() { kernel(__VA_ARGS__); })
/* a launch with start and stop events: the emulator times nothing */
#define hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, e0, e1, flags, ...) \
  simt::launch(dim3(grid), dim3(block), [&]() { kernel(__VA_ARGS__); })
