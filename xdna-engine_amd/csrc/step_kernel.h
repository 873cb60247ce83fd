// step_kernel.h -- the persistent decode-step kernel (device side).
//
// One launch runs every phase of a token.  Each workgroup walks the phase
// list; phase i's virtual blocks are dealt round-robin over the grid, and a
// workgroup waits for phase i's inputs only after issuing the weight loads it
// can (GEMV phases prefetch their first chunks first), so HBM latency
// overlaps the synchronisation.
//
// Synchronisation between phases: each workgroup owns one 128-byte flag slot
// and stores "phases completed" into it (an agent-scope relaxed atomic store
// after s_waitcnt, so its outputs are globally visible first); a waiter polls
// every slot in parallel (thread t polls slot t).  Measured on MI355X: 1.5 us
// per barrier across 256 workgroups, versus 3.9 us for one shared counter
// (atomics serialise at ~11 ns each) and 9.4 us with device-scope fences.
// Activations cross XCDs inside the launch, and the XCDs' L2s are not
// coherent with each other, so every phase reads activations with sc1 loads
// and writes them with agent-scope stores (COH = true in gemv_dev.h /
// attn_dev.h).  Everything a phase body calls is inlined: a real call makes
// the compiler wait for every load in flight, which would cancel the weight
// prefetch issued before the barrier wait.
//
// Flags are never reset: a launch starts from the value in its own slot
// (every slot ends a launch equal), so graph replays need no memset.  A wait
// that exceeds kTimeoutTicks of the device wall clock sets status[0] and every
// workgroup leaves; the host reports the error and re-zeroes the flags.
#pragma once

#include "step_dev.h"

namespace xe {
namespace skern {

using sdev::Phase;

constexpr int kStepThreads = 256;
constexpr uint64_t kTimeoutTicks = 100ull * 1000 * 1000 / 10;  // 100 ms at the 100 MHz wall clock

__device__ __forceinline__ unsigned ld_flag(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Sync {
  unsigned *flags;
  unsigned *status;
  unsigned base;
  int nwg;
  // this workgroup has finished `done` phases: publish after its stores land
  __device__ __forceinline__ void arrive(unsigned done, uint64_t *tr) const {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      if (tr) tr[1] = wall_clock64();
      __hip_atomic_store(flags + 32 * blockIdx.x, base + done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // wait until every workgroup has finished `need` phases; false on timeout
  __device__ __forceinline__ bool wait(unsigned need) const {
    __shared__ int s_bad;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    const unsigned target = base + need;
    const uint64_t t0 = wall_clock64();
    for (int w = threadIdx.x; w < nwg; w += kStepThreads) {
      unsigned spins = 0;
      while (static_cast<int>(ld_flag(flags + 32 * w) - target) < 0) {
        if ((++spins & 255) == 0) {
          if (wall_clock64() - t0 > kTimeoutTicks ||
              __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_bad = 1;
            break;
          }
        }
      }
    }
    __syncthreads();
    return !s_bad;
  }
};

template <int WT, int NB, bool COH, typename Wait>
__device__ __forceinline__ void gemv_phase(const Phase &ph, float4 *lds4, float *red, int first, int stride, Wait wait) {
  using gdev::gemv_tiles;
  const bool writer = first == 0;
#define XE_T(L, R)                                                                          \
  if (ph.lpr == L && ph.rpl == R) {                                                         \
    gemv_tiles<WT, NB, L, R, 4, COH>(ph.u.gemv, lds4, red, first, stride, writer, wait);    \
    return;                                                                                 \
  }
  XE_T(8, 2) XE_T(16, 2) XE_T(16, 1) XE_T(32, 2) XE_T(32, 1) XE_T(64, 2) XE_T(64, 1)
#undef XE_T
  wait();
}

// trace (optional): per phase and workgroup, the device wall clock when the
// phase's inputs were ready and when its outputs were published.
template <int WT, int NB, int HD, int G>
__global__ __launch_bounds__(kStepThreads) void step_kernel(const Phase *phases, int nphases,
                                                            unsigned *flags, unsigned *status,
                                                            uint64_t *trace) {
  extern __shared__ float4 lds4[];
  __shared__ float red[2 * 4 * gdev::kMaxWaves];
  float *lds = reinterpret_cast<float *>(lds4);
  Sync sync{flags, status, ld_flag(flags + 32 * blockIdx.x), static_cast<int>(gridDim.x)};
  bool ok = true;
  for (int i = 0; i < nphases && ok; i++) {
    const Phase &ph = phases[i];
    uint64_t *tr = trace ? trace + 2 * (static_cast<size_t>(i) * gridDim.x + blockIdx.x) : nullptr;
    auto wait = [&]() {
      if (i > 0) ok = sync.wait(static_cast<unsigned>(i));
      if (tr && threadIdx.x == 0) tr[0] = wall_clock64();
    };
    const int first = blockIdx.x, stride = gridDim.x;
    switch (ph.kind) {
      case sdev::PH_GEMV:
        gemv_phase<WT, NB, true>(ph, lds4, red, first, stride, wait);
        break;
      case sdev::PH_ATTN:
        wait();
        if (!ok) break;
        for (int vb = first; vb < ph.nblocks; vb += stride) {
          const adev::AttnParams &a = ph.u.attn;
          const int split = vb % a.max_splits, rest = vb / a.max_splits;
          if (ph.g == G)
            adev::attn_split_block<HD, G, true>(a, split, rest % a.hkv, rest / a.hkv, lds);
          else
            adev::attn_split_block<HD, 1, true>(a, split, rest % a.hkv, rest / a.hkv, lds);
        }
        break;
      case sdev::PH_MERGE:
        wait();
        if (!ok) break;
        for (int vb = first; vb < ph.nblocks; vb += stride) {
          const adev::AttnParams &a = ph.u.attn;
          const int per = (ph.g * HD + kStepThreads - 1) / kStepThreads;
          const int blk = vb % per, rest = vb / per;
          if (ph.g == G)
            adev::attn_merge_block<HD, G, true>(a, blk, rest % a.hkv, rest / a.hkv, lds);
          else
            adev::attn_merge_block<HD, 1, true>(a, blk, rest % a.hkv, rest / a.hkv, lds);
        }
        break;
      case sdev::PH_EMBED:
        wait();
        for (int vb = first; vb < ph.nblocks && ok; vb += stride) sdev::embed_block<true>(ph.u.emb, vb);
        break;
      case sdev::PH_ARGMAX_PART:
        wait();
        for (int vb = first; vb < ph.nblocks && ok; vb += stride) sdev::argmax_part_block<true>(ph.u.arg, vb, lds);
        break;
      case sdev::PH_ARGMAX_FINAL:
        wait();
        for (int vb = first; vb < ph.nblocks && ok; vb += stride) sdev::argmax_final_block<true>(ph.u.arg, vb);
        break;
    }
    if (ok) sync.arrive(static_cast<unsigned>(i + 1), tr);
  }
}

using StepFn = void (*)(const Phase *, int, unsigned *, unsigned *, uint64_t *);

template <int WT, int NB>
StepFn pick_head(int hd, int g) {
  if (hd == 64 && g == 1) return step_kernel<WT, NB, 64, 1>;
  if (hd == 256 && g == 4) return step_kernel<WT, NB, 256, 4>;
  return nullptr;
}

template <int WT>
StepFn pick_nb(int nb, int hd, int g) {
  switch (nb) {
    case 1: return pick_head<WT, 1>(hd, g);
    case 2: return pick_head<WT, 2>(hd, g);
    case 4: return pick_head<WT, 4>(hd, g);
  }
  return nullptr;
}

// One translation unit per weight dtype instantiates the kernels (step_i8.hip,
// step_bf16.hip, step_bfp16.hip) so they compile in parallel.
StepFn pick_step_i8(int nb, int hd, int g);
StepFn pick_step_bf16(int nb, int hd, int g);
StepFn pick_step_bfp16(int nb, int hd, int g);

}  // namespace skern
}  // namespace xe
