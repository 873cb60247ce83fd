// attn.hip -- split-K flash-decode attention kernels for gfx950 (device code
// in attn_dev.h): a partial launch over (split, kv head, stream) and a merge
// launch over (element block, kv head, stream).
#include <mutex>

#include "step_dev.h"

namespace xe {
namespace adev {

AttnParams to_params(const AttnLaunch &L) {
  AttnParams p{};
  p.q = L.q;
  p.q_stride = L.q_stride ? L.q_stride : L.hq * L.hd;
  p.kc = L.kc;
  p.vc = L.vc;
  p.kv_bstride = L.kv_batch_stride;
  p.max_ctx = L.max_ctx;
  p.batch = L.batch;
  p.hq = L.hq;
  p.hkv = L.hkv;
  p.scale = L.scale;
  p.lens = L.lens;
  p.pos = L.pos;
  p.fixed_len = L.fixed_len;
  p.k_new = L.k_new;
  p.v_new = L.v_new;
  p.kv_new_stride = L.kv_new_stride;
  p.q_norm_w = L.q_norm_w;
  p.k_norm_w = L.k_norm_w;
  p.norm_eps = L.norm_eps;
  p.rope_cos = L.rope_cos;
  p.rope_sin = L.rope_sin;
  p.div_norm = L.div_norm;
  p.out = L.out;
  p.out_stride = L.out_stride ? L.out_stride : L.hq * L.hd;
  p.work = L.work;
  p.max_splits = L.max_splits;
  p.k_scale = L.k_scale;
  p.v_scale = L.v_scale;
  p.cnt = L.cnt;
  return p;
}

}  // namespace adev

namespace {

using adev::AttnParams;
using adev::kThreads;

// NT: nontemporal key / value loads (per-stream caches; false for a cache
// every stream of the batch reads).
template <int HD, int G, int KV8 = 0, bool NT = true>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnParams p) {
  __shared__ float lds[adev::attn_lds_floats(HD, G)];
  adev::attn_split_block<HD, G, false, KV8, NT>(p, blockIdx.x, blockIdx.y, blockIdx.z, lds);
}

template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnParams p) {
  __shared__ float lds[adev::merge_lds_floats()];
  adev::attn_merge_block<HD, G, false>(p, blockIdx.x, blockIdx.y, blockIdx.z, lds);
}

using AttnFn = void (*)(AttnParams);

template <int HD>
AttnFn pick_g(int g, bool merge, bool shared) {
  switch (g) {
    case 1: return merge ? attn_merge_kernel<HD, 1> : shared ? attn_kernel<HD, 1, 0, false> : attn_kernel<HD, 1>;
    case 2: return merge ? attn_merge_kernel<HD, 2> : attn_kernel<HD, 2>;
    case 4: return merge ? attn_merge_kernel<HD, 4> : attn_kernel<HD, 4>;
    case 8: return merge ? attn_merge_kernel<HD, 8> : attn_kernel<HD, 8>;
  }
  return nullptr;
}

// int8 K and/or V (kv8 bit 0 / bit 1): one query head a KV head (Whisper's
// cross attention, its cache shared by the batch: plain loads).
template <int HD>
AttnFn pick_kv8(int kv8) {
  switch (kv8) {
    case 1: return attn_kernel<HD, 1, 1, false>;
    case 2: return attn_kernel<HD, 1, 2, false>;
    case 3: return attn_kernel<HD, 1, 3, false>;
  }
  return nullptr;
}

// shared: one K / V cache for every stream of the batch (batch stride 0),
// which then loads with plain loads (one query head a KV head: cross
// attention; other groups keep the nontemporal kernel).
AttnFn pick(int hd, int g, bool merge, int kv8 = 0, bool shared = false) {
  if (kv8 && !merge) {
    if (g != 1) return nullptr;
    switch (hd) {
      case 64: return pick_kv8<64>(kv8);
      case 128: return pick_kv8<128>(kv8);
      case 256: return pick_kv8<256>(kv8);
    }
    return nullptr;
  }
  switch (hd) {
    case 64: return pick_g<64>(g, merge, shared);
    case 128: return pick_g<128>(g, merge, shared);
    case 256: return pick_g<256>(g, merge, shared);
  }
  return nullptr;
}

int kv8_of(const AttnParams &p) { return (p.k_scale ? 1 : 0) | (p.v_scale ? 2 : 0); }

}  // namespace

// One attention phase of a step: split partials or the merge (none with
// arrival counters: the split kernel merges in place).
void launch_attn_phase(const sdev::Phase &ph, hipStream_t s) {
  const AttnParams &p = ph.u.attn;
  const bool merge = ph.kind == sdev::PH_MERGE;
  if (merge && p.cnt) return;
  AttnFn fn = pick(ph.hd, ph.g, merge, kv8_of(p), p.kv_bstride == 0 && p.batch > 1);
  XE_REQUIRE(fn, "attn phase: unsupported head_dim / group (int8 K/V: one query head a KV head)");
  if (merge) {
    const int blocks = (ph.g * ph.hd + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(fn, dim3(blocks, p.hkv, p.batch), dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL(fn, dim3(p.max_splits, p.hkv, p.batch), dim3(kThreads), 0, s, p);
  }
  XE_HIP(hipGetLastError());
}

size_t attn_work_floats(int batch, int hq, int hd, int max_splits) {
  return static_cast<size_t>(batch) * hq * max_splits * (hd + 2);
}

// ---------------------------------------------------------------------------
// Workspace of the allocation-free entry point (xe_attn_decode_dev_static):
// the split partials live in this file-scope device array, one copy per GPU
// for the life of the process.  In host code `scratch` is only a stand-in
// symbol: its device address comes from hipGetSymbolAddress, resolved once
// per device with that device current, and only that address is ever passed
// to kernels.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kStaticAttnFloats = size_t(4) << 20;  // 16 MB of partials
__device__ __align__(256) float scratch[kStaticAttnFloats];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

size_t attn_static_floats() { return kStaticAttnFloats; }

void *attn_static_scratch(int ordinal) {
  XE_REQUIRE(ordinal >= 0 && ordinal < kMaxDevices, "device ordinal out of range for the static workspace");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[ordinal]) {
    DeviceGuard dg(ordinal);
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    XE_REQUIRE(e == hipSuccess && ptr, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[ordinal] = ptr;
  }
  return g_scratch_ptr[ordinal];
}

void launch_attn(const AttnLaunch &L, hipStream_t s) {
  XE_REQUIRE(L.batch > 0 && L.hq > 0 && L.hkv > 0 && L.hq % L.hkv == 0, "attn: bad heads");
  XE_REQUIRE(L.max_ctx > 0, "attn: max_ctx must be > 0");
  XE_REQUIRE(L.max_splits >= 1 && L.max_splits <= adev::kMaxSplits, "attn: max_splits must be 1..256");
  XE_REQUIRE(L.work, "attn: workspace missing");
  const int g = L.hq / L.hkv;
  const AttnParams p = adev::to_params(L);
  AttnFn fn = pick(L.hd, g, false, kv8_of(p), p.kv_bstride == 0 && p.batch > 1);
  AttnFn merge = pick(L.hd, g, true);
  XE_REQUIRE(fn && merge, "attn: unsupported head_dim / GQA group (hd 64/128/256, group 1/2/4/8; "
                          "int8 K/V: group 1)");
  XE_REQUIRE(!L.rope_cos || (L.rope_sin && L.pos), "attn: RoPE needs sin table and positions");
  XE_REQUIRE(!L.k_new || (L.v_new && (L.pos || L.lens || L.fixed_len)), "attn: append needs v_new");
  XE_REQUIRE(!kv8_of(p) || !L.k_new, "attn: int8 K/V caches take no append");
  hipLaunchKernelGGL(fn, dim3(L.max_splits, L.hkv, L.batch), dim3(kThreads), 0, s, p);
  XE_HIP(hipGetLastError());
  if (L.max_splits > 1 && !L.cnt) {
    const int blocks = (g * L.hd + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(merge, dim3(blocks, L.hkv, L.batch), dim3(kThreads), 0, s, p);
    XE_HIP(hipGetLastError());
  }
}

}  // namespace xe
