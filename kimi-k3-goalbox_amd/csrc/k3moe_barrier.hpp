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
// invalidates the local L2 for the reads that follow.
struct BarrierBase {
  unsigned top, grp;  // the top counter and this workgroup's group counter before barrier 1
};

__device__ __forceinline__ unsigned bar_groups() { return gridDim.x < kBarGroups ? gridDim.x : kBarGroups; }

// Thread 0, at the kernel's start: no barrier of this launch can complete
// before this workgroup arrives, so the counters hold whole barriers of
// earlier launches plus arrivals of this launch's barrier 1 (fewer than a
// group's members, or fewer than all groups); rounding down removes those.
__device__ __forceinline__ BarrierBase barrier_base(const unsigned *ctl) {
  const unsigned groups = bar_groups(), members = gridDim.x / groups, g = blockIdx.x % groups;
  const unsigned t = __hip_atomic_load(ctl + kCtlTop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned c = __hip_atomic_load(ctl + kCtlGroup + g * kCtlStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return BarrierBase{t & ~(groups - 1u), c & ~(members - 1u)};
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

// Thread 0: spins until the top counter shows every group (bounded: a timeout
// or another workgroup's error ends it), then acquires at agent scope.
__device__ __forceinline__ void barrier_wait(unsigned *ctl, const BarrierBase &bb, unsigned n, uint64_t *trace) {
  const unsigned target = bb.top + n * bar_groups();
  unsigned spins = 0;
  while ((int)(__hip_atomic_load(ctl + kCtlTop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
    if ((++spins & 63u) == 0u) {
      if (__hip_atomic_load(ctl + kCtlErr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
      if (spins > kSpinLimit) {
        __hip_atomic_store(ctl + kCtlErr, (unsigned)kErrBarrierTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  if (trace) trace[2] = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (trace) trace[3] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void grid_barrier(unsigned *ctl, const BarrierBase &bb, unsigned n,
                                             uint64_t *trace = nullptr) {
  wait_vmem();  // this wave's device-coherent stores are done (and thread 0's base loads)
  __syncthreads();
  if (threadIdx.x == 0) {
    barrier_arrive(ctl, bb, n, trace);
    barrier_wait(ctl, bb, n, trace);
  }
  __syncthreads();
}

}  // namespace k3moe
