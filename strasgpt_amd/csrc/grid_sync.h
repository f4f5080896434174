// Grid-wide barrier for kernels whose blocks are all resident at once
// (launched with no more blocks than the device holds at the kernel's
// occupancy).
//
// Arrival is by flags, not by a shared counter: atomics on one address are
// serialised by the memory side (about 65 ns each on MI355X, so 17 us for
// 256 arrivals), while stores to distinct lines proceed in parallel. Each
// block stores the barrier's sequence number into its own 128-byte slot;
// block 0 waits for all slots (one thread per slot), then stores the number
// into the `go` line, which the other blocks poll.
//
// The sequence number is kept by the caller (`GridSync::seq`, the same in
// every block, incremented by each barrier) and starts at `base`, a value
// larger than any left in the state words by earlier launches: the host
// passes a per-launch base (see `grid_sync_base`), so the state never needs
// clearing between launches.
//
// Every wait is bounded: a block that sees no progress for `kSyncTimeoutTicks`
// of the 100 MHz wall clock records 1 in err[0] and leaves the barrier;
// once err[0] is set no block waits at any barrier, so the kernel always
// finishes. The host checks err[0] after the launch and treats a set flag as
// fatal (the results of that launch are invalid).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sg {

constexpr uint64_t kSyncTimeoutTicks = 20000000;  // 200 ms at 100 MHz
constexpr int kSyncSlotWords = 32;                // 128-byte slot per block
constexpr int kSyncMaxBlocks = 1024;

// Device state: `go` line, then one slot per block.
constexpr size_t kSyncStateWords = kSyncSlotWords * (1 + kSyncMaxBlocks);

struct GridSync {
  unsigned* state;  // kSyncStateWords words
  unsigned* err;    // [1], set to 1 on a timed-out wait
  unsigned seq;     // sequence number of the next barrier
};

__device__ __forceinline__ unsigned sync_load(const unsigned* p) {
  return __hip_atomic_load((const __attribute__((address_space(1))) unsigned*)p, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(unsigned* p, unsigned v) {
  __hip_atomic_store((__attribute__((address_space(1))) unsigned*)p, v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until *p reaches `want` (wrap-safe), or the error flag is set or the
// wait times out. Returns false on error or time-out.
__device__ __forceinline__ bool sync_wait(const unsigned* p, unsigned want, unsigned* err) {
  const uint64_t t0 = wall_clock64();
  while ((int)(sync_load(p) - want) < 0) {
    __builtin_amdgcn_s_sleep(2);
    if (sync_load(err)) return false;
    if (wall_clock64() - t0 > kSyncTimeoutTicks) {
      sync_store(err, 1u);
      return false;
    }
  }
  return true;
}

// s_waitcnt operand: at most `vm` vector memory operations outstanding,
// no LDS/scalar operation outstanding.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | (7 << 4) | (0 << 8) | ((vm >> 4) << 14); }

// Workgroup barrier that lets each wave keep its newest `PENDING` vector
// memory operations in flight (gfx9 completes them in issue order, so every
// older one, stores included, has completed). The empty asm statements keep
// the compiler from moving memory accesses across the barrier.
template <int PENDING>
__device__ __forceinline__ void block_barrier_pending() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool FENCE, int PENDING>
__device__ __forceinline__ void grid_sync_impl(GridSync& g) {
  const unsigned seq = g.seq++;
  unsigned* go = g.state;
  unsigned* slot = g.state + kSyncSlotWords;
  if (FENCE)
    __syncthreads();
  else
    block_barrier_pending<PENDING>();
  if (threadIdx.x == 0) {
    if (FENCE) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    sync_store(slot + blockIdx.x * kSyncSlotWords, seq);
  }
  if (blockIdx.x == 0) {
    for (unsigned b = threadIdx.x; b < gridDim.x; b += blockDim.x)
      if (!sync_wait(slot + b * kSyncSlotWords, seq, g.err)) break;
    if (FENCE)
      __syncthreads();
    else
      block_barrier_pending<PENDING>();
    if (threadIdx.x == 0) {
      if (FENCE) __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "agent");
      sync_store(go, seq);
    }
  } else if (threadIdx.x == 0) {
    sync_wait(go, seq, g.err);
  }
  if (threadIdx.x == 0 && FENCE) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (FENCE)
    __syncthreads();
  else
    block_barrier_pending<PENDING>();
}

// FENCE = true: every store issued by any block before the call is visible
// to every block after it returns (agent-scope release before arrival,
// acquire after). FENCE = false: only stores made with `sync_store` (or
// other agent-scope atomics) before the call are visible after it, to
// loads made with `sync_load`; the barrier waits for them to complete
// before the block's arrival is stored.
template <bool FENCE = true>
__device__ __forceinline__ void grid_sync(GridSync& g) {
  grid_sync_impl<FENCE, 0>(g);
}

// Fence-free barrier (as grid_sync<false>) for a block whose waves have
// each issued at least `PENDING` vector loads after their last store that
// must be visible: the newest `PENDING` of them stay in flight through the
// barrier (weights of the next phase, typically).
template <int PENDING>
__device__ __forceinline__ void grid_sync_pending(GridSync& g) {
  grid_sync_impl<false, PENDING>(g);
}

// Split barrier for a grid of one master block (index 0), which does
// nothing but coordinate, and worker blocks (1 .. gridDim.x - 1), which
// arrive as soon as their stores are complete and may issue loads for the
// next phase before waiting:
//   worker: stores ... grid_arrive(g); next-phase loads ...; grid_wait(g);
//   master: grid_master(g);
// Visibility is that of grid_sync<false>: stores made with `sync_store`
// before grid_arrive are seen by `sync_load`s after grid_wait.
__device__ __forceinline__ void grid_arrive(const GridSync& g) {
  block_barrier_pending<0>();
  if (threadIdx.x == 0) sync_store(g.state + kSyncSlotWords * (1 + blockIdx.x), g.seq);
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void grid_wait(GridSync& g) {
  if (threadIdx.x == 0) sync_wait(g.state, g.seq, g.err);
  block_barrier_pending<63>();  // no wait for vector memory operations
  g.seq++;
}

__device__ __forceinline__ void grid_master(GridSync& g) {
  unsigned* slot = g.state + kSyncSlotWords;
  for (unsigned b = 1 + threadIdx.x; b < gridDim.x; b += blockDim.x)
    if (!sync_wait(slot + b * kSyncSlotWords, g.seq, g.err)) break;
  block_barrier_pending<0>();
  if (threadIdx.x == 0) sync_store(g.state, g.seq);
  g.seq++;
}

}  // namespace sg
