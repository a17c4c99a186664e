// Grid barrier of the persistent kernels (decode step, latent block): all
// workgroups of a launch meet; data written before it with device-coherent
// stores is visible to every workgroup after it.
#pragma once

#include "k3moe_device.hpp"
#include "k3moe_plan.hpp"

namespace k3moe {

constexpr unsigned kSpinLimit = 1u << 21;  // bounded barrier wait (about 0.1-1 s)

// Grid barrier number `n` (1-based) of this launch over gridDim.x (a power of
// two) workgroups. Arrival is two-level so that no counter sees more than
// kBarGroups arrivals per barrier: workgroup b counts in on group counter
// b mod kBarGroups; the last arrival of a group counts the group in on the top
// counter. The counters are never reset: `bb` holds their values before this
// launch's first barrier, and every count is a power of two, so the 32-bit
// wrap keeps whole barriers whole. Data that crosses a barrier is written with
// device-coherent stores (st_dev*), so arriving needs only their completion
// (every wave waits for its vector memory operations) and a relaxed
// increment; after the top counter shows every group, an agent-scope acquire
// invalidates the local L2 for the reads that follow, unless the caller reads
// the barrier's data only with device-coherent loads (acquire = false): the
// invalidation takes microseconds and empties the XCD's L2 for every
// workgroup on it.
struct BarrierBase {
  unsigned top, grp;  // the top counter and this workgroup's group counter before barrier 1
  unsigned abort;     // the abort counter at this workgroup's start
};

// A wait of this launch gave up: record it in the sticky status word and move
// the abort counter, so that the launch's other waits stop early.
__device__ __forceinline__ void raise_timeout(unsigned *ctl) {
  __hip_atomic_fetch_or(ctl + kCtlErr, (unsigned)kErrBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(ctl + kCtlAbort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A launch that gave up a wait leaves NaN in its output, so that a caller
// that does not read the status word still cannot take it for a result: each
// workgroup that gave up, or that ends after another one did, fills its share
// [n b / G, n (b + 1) / G) of the output's n elements (fp32, or bf16 when
// BF16). Kernels call it from every thread.
template <bool BF16>
__device__ __forceinline__ void poison_share(void *out, long n) {
  const long lo = n * (long)blockIdx.x / (long)gridDim.x, hi = n * ((long)blockIdx.x + 1) / (long)gridDim.x;
  for (long j = lo + threadIdx.x; j < hi; j += blockDim.x) {
    if (BF16) reinterpret_cast<uint16_t *>(out)[j] = 0x7FC0u;
    else reinterpret_cast<uint32_t *>(out)[j] = 0x7FC00000u;
  }
}

// The abort counter moved since `base`: a wait of this launch gave up.
__device__ __forceinline__ bool aborted(const unsigned *ctl, unsigned base) {
  return __hip_atomic_load(ctl + kCtlAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != base;
}

__device__ __forceinline__ unsigned bar_groups() { return gridDim.x < kBarGroups ? gridDim.x : kBarGroups; }

// Thread 0, at the kernel's start: no barrier of this launch can complete
// before this workgroup arrives, so the counters hold whole barriers of
// earlier launches plus arrivals of this launch's barrier 1 (fewer than a
// group's members, or fewer than all groups); rounding down removes those.
__device__ __forceinline__ BarrierBase barrier_base(const unsigned *ctl) {
  const unsigned groups = bar_groups(), members = gridDim.x / groups, g = blockIdx.x % groups;
  const unsigned t = __hip_atomic_load(ctl + kCtlTop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned c = __hip_atomic_load(ctl + kCtlGroup + g * kCtlStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned ab = __hip_atomic_load(ctl + kCtlAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return BarrierBase{t & ~(groups - 1u), c & ~(members - 1u), ab};
}

// Thread 0's arrival: counts this workgroup in on its group counter, and the
// group in on the top counter when it is the group's last.
__device__ __forceinline__ void barrier_arrive(unsigned *ctl, const BarrierBase &bb, unsigned n, uint64_t *trace) {
  const unsigned groups = bar_groups(), members = gridDim.x / groups, g = blockIdx.x % groups;
  if (trace) trace[0] = __builtin_amdgcn_s_memrealtime();
  const unsigned old = __hip_atomic_fetch_add(ctl + kCtlGroup + g * kCtlStride, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
  if (old == bb.grp + n * members - 1u)
    __hip_atomic_fetch_add(ctl + kCtlTop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (trace) trace[1] = __builtin_amdgcn_s_memrealtime();
}

// Thread 0: spins until the top counter shows every group, then (acquire)
// acquires at agent scope. Bounded: it gives up after kSpinLimit polls (a timeout), or
// when another wait of this launch gave up. Returns false when it gave up.
__device__ __forceinline__ bool barrier_wait(unsigned *ctl, const BarrierBase &bb, unsigned n, uint64_t *trace,
                                             bool acquire = true) {
  const unsigned target = bb.top + n * bar_groups();
  unsigned spins = 0;
  bool ok = true;
  while ((int)(__hip_atomic_load(ctl + kCtlTop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
    if ((++spins & 63u) == 0u) {
      if (aborted(ctl, bb.abort)) {
        ok = false;
        break;
      }
      if (spins > kSpinLimit) {
        raise_timeout(ctl);
        ok = false;
        break;
      }
    }
  }
  if (trace) trace[2] = __builtin_amdgcn_s_memrealtime();
  if (acquire) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (trace) trace[3] = __builtin_amdgcn_s_memrealtime();
  return ok;
}

// Returns false in every thread of the workgroup when the wait gave up: the
// data the barrier should publish may be incomplete, so the caller leaves
// (every later wait of the launch then gives up early too).
__device__ __forceinline__ bool grid_barrier(unsigned *ctl, const BarrierBase &bb, unsigned n,
                                             uint64_t *trace = nullptr, bool acquire = true) {
  __shared__ int s_ok;
  wait_vmem();  // this wave's device-coherent stores are done (and thread 0's base loads)
  __syncthreads();
  if (threadIdx.x == 0) {
    barrier_arrive(ctl, bb, n, trace);
    s_ok = barrier_wait(ctl, bb, n, trace, acquire) ? 1 : 0;
  }
  __syncthreads();
  return s_ok != 0;
}

// Launch tags of the single-token and decode kernels number their launches
// modulo 2^32 / G (the launch counters' sum over the grid size G, plus one),
// so a slot that no launch wrote for a whole cycle would carry a current tag.
// The last launch of each cycle (tag 2^32 / G) therefore ends with a grid
// barrier, after which each workgroup zeroes its share of the tag area: every
// launch of the next cycle then finds slots written in that cycle or zeros
// (which no tag matches).
// Code warm-up of a persistent kernel whose last launch recorded its code
// range [range[0], range[1]) (the program counter at its start and near its
// end): at a launch with the same start every workgroup loads a slice of the
// range as data (wave w of workgroup b: 1 KiB chunk b / 8 + 32 w, so the 32
// workgroups of an XCD cover up to 256 KiB of its L2), so that the kernel's
// first instruction fetches of each stretch of code hit L2 instead of queueing
// for HBM behind its own weight loads. Loads only inside the recorded range
// (the kernel's own first bytes otherwise); the caller keeps the returned
// value live until the loads may complete. Waits for the range words first.
__device__ __forceinline__ u32x4 warm_code_range(const uint64_t *range, uint64_t pc0) {
  const uint64_t c0 = range[0], c1 = range[1];
  u32x4 v = {0, 0, 0, 0};
  if (c0 == pc0 && c1 > pc0 && c1 - pc0 < (1u << 20)) {
    const uint64_t lo = pc0 & ~(uint64_t)1023;
    const uint64_t addr = lo + (uint64_t)((blockIdx.x >> 3) + 32 * (threadIdx.x >> 6)) * 1024 + (threadIdx.x & 63) * 16;
    const uint64_t at = addr + 16 <= c1 ? addr : (pc0 & ~(uint64_t)15);
    v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(at);
  }
  return v;
}

__device__ __forceinline__ uint32_t last_tag_of_cycle() {
  return (uint32_t)(0x100000000ull >> __builtin_ctz(gridDim.x));
}

// Barrier `n` of the launch, then this workgroup's share of the tag area
// cleared with device-coherent stores (the next launch polls it with
// device-coherent loads). Returns false when the barrier's wait gave up.
__device__ __forceinline__ bool clear_tag_area(unsigned *ctl, const BarrierBase &bb, unsigned n,
                                               __amdgpu_buffer_rsrc_t tagr) {
  if (!grid_barrier(ctl, bb, n, nullptr, false)) return false;
  const uint32_t share = (uint32_t)kTagBytes / gridDim.x;  // a multiple of 16 (G <= 1024)
  for (uint32_t off = blockIdx.x * share + threadIdx.x * 16; off < (blockIdx.x + 1) * share; off += blockDim.x * 16)
    st_dev128(tagr, off, u32x4{0u, 0u, 0u, 0u});
  return true;
}

}  // namespace k3moe
