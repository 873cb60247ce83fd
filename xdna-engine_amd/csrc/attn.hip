// attn.hip -- single-query attention over a bf16 KV cache (split-K flash
// decode) for gfx950.
//
// Replaces the reference's mha_decode (route_b_kernels/mha_decode/
// mha_decode.cc:90-175: online softmax per key over streamed K/V tiles with a
// runtime key count) and its host driver CtxDecode::attn
// (rust/npu-asr/src/ctx_decode.rs:468-555), generalised to GQA, head_dim
// 64/128/256, per-stream lengths and contexts far beyond the reference's 448.
// The arithmetic target is attend_one (whisper_decoder.rs:242-278): scores
// (q.k) * scale in fp32, softmax, p-weighted sum of V.
//
// Grid (split, kv_head, stream).  Each workgroup takes one contiguous key
// range of one (stream, kv head) and all G = hq/hkv query heads that share it,
// so the K/V bytes of a GQA group are read once.  Inside the workgroup:
//   * L = hd/8 lanes hold one key (16 B of bf16 each); a wave reads 64/L
//     consecutive keys per load: whole 128-byte lines.
//   * Each lane group keeps an online-softmax state (m, l, acc) per query head
//     in registers, updated once per block of UK keys (log2 domain, exp2).
//   * Lane groups merge by xor-shuffles, waves through LDS; the workgroup
//     writes (m, l, acc) to the workspace (or the output when one split
//     covers the whole length).
//   * A second small launch merges the splits of each (stream, kv head).
//     (A last-arriving-workgroup merge needs device-scope release/acquire
//     fences, which write back and invalidate L2 on this part and measured
//     ~80 us per launch; the kernel boundary is cheaper.)
// Fused in front (decode step): the Gemma per-head RMSNorm (1 + w) and RoPE of
// q and the new k, and the bf16 append of the new k/v at position pos, done
// by the workgroup whose range holds pos (the only one that reads it).
#include "common.h"

namespace xe {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMinChunk = 64;  // keys per split at least (amortises per-workgroup setup)

struct AttnParams {
  const float *q;
  int q_stride;
  uint16_t *kc, *vc;
  size_t kv_bstride;
  int max_ctx;
  int batch, hq, hkv;
  float scale;
  const int32_t *lens;
  const int32_t *pos;
  int fixed_len;
  const float *k_new, *v_new;
  int kv_new_stride;
  const float *q_norm_w, *k_norm_w;
  float norm_eps;
  const float *rope_cos, *rope_sin;
  int div_norm;
  float *out;
  int out_stride;
  float *work;
  int max_splits;
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  // Integer RNE with quiet-NaN, bit-identical to f32_to_bf16_bits
  // (rust/npu-xrt/src/lib.rs:809-817).
  uint32_t bits = __float_as_uint(x);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x0040u);
  uint32_t bias = 0x00007fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>((bits + bias) >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ int stream_len(const AttnParams &p, int b) {
  if (p.lens) return p.lens[b];
  if (p.pos) return p.pos[b] + 1;
  return p.fixed_len;
}

__device__ __forceinline__ void split_range(int len, int max_splits, int &chunk, int &nsplits) {
  int per = (len + max_splits - 1) / max_splits;
  per = (per + kMinChunk - 1) / kMinChunk * kMinChunk;
  chunk = per < kMinChunk ? kMinChunk : per;
  nsplits = (len + chunk - 1) / chunk;
}

// Per-head RMSNorm (1+w) and RoPE on one head vector held by one wave:
// lane j (< hd/2) owns elements (j, j + hd/2) for j = lane, lane + 64, ...
template <int HD>
__device__ void head_transform(const AttnParams &p, const float *src, float *dst,
                               const float *norm_w, int posi) {
  constexpr int HALF = HD / 2;
  constexpr int PER = (HALF + 63) / 64;
  const int lane = threadIdx.x & 63;
  float a[PER], c[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = lane + 64 * i;
    a[i] = j < HALF ? src[j] : 0.f;
    c[i] = j < HALF ? src[j + HALF] : 0.f;
    ss = ss + a[i] * a[i];
    ss = ss + c[i] * c[i];
  }
  if (norm_w) {
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(HD) + p.norm_eps);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int j = lane + 64 * i;
      if (j < HALF) {
        a[i] = a[i] * inv * (1.0f + norm_w[j]);
        c[i] = c[i] * inv * (1.0f + norm_w[j + HALF]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = lane + 64 * i;
    if (j >= HALF) continue;
    float x0 = a[i], x1 = c[i];
    if (p.rope_cos) {
      const float cs = p.rope_cos[static_cast<size_t>(posi) * HALF + j];
      const float sn = p.rope_sin[static_cast<size_t>(posi) * HALF + j];
      // rotate_half pairing (npu-asr-host/src/lib.rs:143-185)
      const float y0 = x0 * cs - x1 * sn;
      const float y1 = x1 * cs + x0 * sn;
      x0 = y0;
      x1 = y1;
    }
    dst[j] = x0;
    dst[j + HALF] = x1;
  }
}

template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnParams p) {
  constexpr int EPL = 8;          // bf16 elements per lane per key (16 B)
  constexpr int L = HD / EPL;     // lanes per key
  constexpr int KPW = 64 / L;     // keys per wave per load
  constexpr int UK = 4;           // keys per lane group per block update
  constexpr int STEP = kWaves * KPW;

  __shared__ float qs[G][HD];
  __shared__ float red[kWaves][G][HD + 2];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int len = stream_len(p, b);
  if (len <= 0) return;
  int chunk, nsplits;
  split_range(len, p.max_splits, chunk, nsplits);
  if (split >= nsplits) return;
  const int s0 = split * chunk;
  const int s1 = min(len, s0 + chunk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int posi = len - 1;

  uint16_t *kbase = p.kc + p.kv_bstride * b + static_cast<size_t>(kvh) * p.max_ctx * HD;
  uint16_t *vbase = p.vc + p.kv_bstride * b + static_cast<size_t>(kvh) * p.max_ctx * HD;

  // ---- q heads of this group (norm + rope), new k/v append ----
  for (int g = wave; g < G; g += kWaves) {
    const float *src = p.q + static_cast<size_t>(b) * p.q_stride + (kvh * G + g) * HD;
    head_transform<HD>(p, src, qs[g], p.q_norm_w, posi);
  }
  const bool appender = p.k_new && split == nsplits - 1;
  if (appender && wave == 0) {
    const float *ksrc = p.k_new + static_cast<size_t>(b) * p.kv_new_stride + kvh * HD;
    const float *vsrc = p.v_new + static_cast<size_t>(b) * p.kv_new_stride + kvh * HD;
    float *kt = red[0][0];  // scratch: transformed k
    head_transform<HD>(p, ksrc, kt, p.k_norm_w, posi);
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < HD; j += 64) {
      kbase[static_cast<size_t>(posi) * HD + j] = f32_to_bf16_rne(kt[j]);
      vbase[static_cast<size_t>(posi) * HD + j] = f32_to_bf16_rne(vsrc[j]);
    }
  }
  __syncthreads();  // the appended row is read back by this workgroup only

  // ---- main loop: online softmax per lane group ----
  const int kg = lane / L, kl = lane % L;
  float qr[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int e = 0; e < EPL; e++) qr[g][e] = qs[g][kl * EPL + e];
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[g][e] = 0.f;
  }
  const float sc2 = p.scale * kLog2e;

  for (int base = s0 + wave * KPW + kg; base < s1; base += STEP * UK) {
    uint4 kv[UK], vv[UK];
    bool ok[UK];
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const int key = base + u * STEP;
      ok[u] = key < s1;
      const int kk = ok[u] ? key : s0;
      kv[u] = *reinterpret_cast<const uint4 *>(kbase + static_cast<size_t>(kk) * HD + kl * EPL);
      vv[u] = *reinterpret_cast<const uint4 *>(vbase + static_cast<size_t>(kk) * HD + kl * EPL);
    }
    float s[UK][G];
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const uint32_t w[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
      float kf[EPL];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kf[2 * i] = __uint_as_float(w[i] << 16);
        kf[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
#pragma unroll
      for (int g = 0; g < G; g++) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) d = __builtin_fmaf(qr[g][e], kf[e], d);
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) d += __shfl_xor(d, off, 64);
        s[u][g] = d * sc2;
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      float mb = m[g];
#pragma unroll
      for (int u = 0; u < UK; u++)
        if (ok[u]) mb = fmaxf(mb, s[u][g]);
      if (mb == -INFINITY) continue;  // no valid key for this group yet
      const float corr = __builtin_amdgcn_exp2f(m[g] - mb);
      float pu[UK];
      float psum = 0.f;
#pragma unroll
      for (int u = 0; u < UK; u++) {
        pu[u] = ok[u] ? __builtin_amdgcn_exp2f(s[u][g] - mb) : 0.f;
        psum += pu[u];
      }
      l[g] = l[g] * corr + psum;
      m[g] = mb;
#pragma unroll
      for (int e = 0; e < EPL; e++) acc[g][e] *= corr;
#pragma unroll
      for (int u = 0; u < UK; u++) {
        const uint32_t w[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          acc[g][2 * i] = __builtin_fmaf(pu[u], __uint_as_float(w[i] << 16), acc[g][2 * i]);
          acc[g][2 * i + 1] =
              __builtin_fmaf(pu[u], __uint_as_float(w[i] & 0xffff0000u), acc[g][2 * i + 1]);
        }
      }
    }
  }

  // ---- merge lane groups inside the wave ----
#pragma unroll
  for (int off = L; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float mo = __shfl_xor(m[g], off, 64);
      const float lo = __shfl_xor(l[g], off, 64);
      const float mx = fmaxf(m[g], mo);
      const float a = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[g] - mx);
      const float c = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mx);
      l[g] = l[g] * a + lo * c;
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        const float ao = __shfl_xor(acc[g][e], off, 64);
        acc[g][e] = acc[g][e] * a + ao * c;
      }
      m[g] = mx;
    }
  }
  if (kg == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
      for (int e = 0; e < EPL; e++) red[wave][g][2 + kl * EPL + e] = acc[g][e];
      if (kl == 0) {
        red[wave][g][0] = m[g];
        red[wave][g][1] = l[g];
      }
    }
  }
  __syncthreads();

  // ---- merge waves: thread t -> (head g, element e) ----
  const bool single = nsplits == 1;
  float *wbase = p.work + (static_cast<size_t>(b) * p.hq + kvh * G) * p.max_splits * (HD + 2);
  for (int t = threadIdx.x; t < G * HD; t += kThreads) {
    const int g = t / HD, e = t % HD;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) mx = fmaxf(mx, red[w][g][0]);
    float lt = 0.f, at = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float mw = red[w][g][0];
      const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
      lt += red[w][g][1] * f;
      at += red[w][g][2 + e] * f;
    }
    if (single) {
      const float o = p.div_norm ? at / lt : at * (1.0f / lt);
      p.out[static_cast<size_t>(b) * p.out_stride + (kvh * G + g) * HD + e] = o;
    } else {
      float *dst = wbase + (static_cast<size_t>(g) * p.max_splits + split) * (HD + 2);
      dst[2 + e] = at;
      if (e == 0) {
        dst[0] = mx;
        dst[1] = lt;
      }
    }
  }
}

// Merge the split partials of one (stream, kv head): weights exp2(m_s - M),
// out = sum_s acc_s * w_s / sum_s l_s * w_s.  Grid (element block, kv head,
// stream): each workgroup finishes 256 of the G*HD outputs.  A separate
// launch: the kernel boundary publishes the partials, so no workgroup needs a
// device-scope fence.
template <int HD, int G>
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnParams p) {
  constexpr int MAXS = 256;
  constexpr int HPB = kThreads >= HD ? kThreads / HD : 1;  // heads per block
  __shared__ float wts[HPB][MAXS];
  __shared__ float lsum[HPB];
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int len = stream_len(p, b);
  if (len <= 0) return;
  int chunk, nsplits;
  split_range(len, p.max_splits, chunk, nsplits);
  if (nsplits == 1) return;  // the partial kernel wrote the output
  const int t0 = blockIdx.x * kThreads;  // first output element of this block
  if (t0 >= G * HD) return;
  const int g0 = t0 / HD;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *wbase = p.work + (static_cast<size_t>(b) * p.hq + kvh * G) * p.max_splits * (HD + 2);
  for (int hh = wave; hh < HPB; hh += kWaves) {
    const int g = g0 + hh;
    if (g >= G) break;
    float mx = -INFINITY;
    for (int sidx = lane; sidx < nsplits; sidx += 64)
      mx = fmaxf(mx, wbase[(static_cast<size_t>(g) * p.max_splits + sidx) * (HD + 2)]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float ls = 0.f;
    for (int sidx = lane; sidx < nsplits; sidx += 64) {
      const float *src = wbase + (static_cast<size_t>(g) * p.max_splits + sidx) * (HD + 2);
      const float ms = src[0];
      const float f = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
      wts[hh][sidx] = f;
      ls += src[1] * f;
    }
    ls = wave_sum(ls);
    if (lane == 0) lsum[hh] = ls;
  }
  __syncthreads();
  const int t = t0 + threadIdx.x;
  if (t >= G * HD) return;
  const int g = t / HD, e = t % HD, hh = g - g0;
  const float *src = wbase + static_cast<size_t>(g) * p.max_splits * (HD + 2) + 2 + e;
  float at0 = 0.f, at1 = 0.f;
  int sidx = 0;
  for (; sidx + 1 < nsplits; sidx += 2) {
    at0 += src[static_cast<size_t>(sidx) * (HD + 2)] * wts[hh][sidx];
    at1 += src[static_cast<size_t>(sidx + 1) * (HD + 2)] * wts[hh][sidx + 1];
  }
  if (sidx < nsplits) at0 += src[static_cast<size_t>(sidx) * (HD + 2)] * wts[hh][sidx];
  const float at = at0 + at1;
  const float o = p.div_norm ? at / lsum[hh] : at * (1.0f / lsum[hh]);
  p.out[static_cast<size_t>(b) * p.out_stride + (kvh * G + g) * HD + e] = o;
}

using AttnFn = void (*)(AttnParams);

template <int HD>
AttnFn pick_g(int g, bool merge) {
  switch (g) {
    case 1: return merge ? attn_merge_kernel<HD, 1> : attn_kernel<HD, 1>;
    case 2: return merge ? attn_merge_kernel<HD, 2> : attn_kernel<HD, 2>;
    case 4: return merge ? attn_merge_kernel<HD, 4> : attn_kernel<HD, 4>;
    case 8: return merge ? attn_merge_kernel<HD, 8> : attn_kernel<HD, 8>;
  }
  return nullptr;
}

AttnFn pick(int hd, int g, bool merge) {
  switch (hd) {
    case 64: return pick_g<64>(g, merge);
    case 128: return pick_g<128>(g, merge);
    case 256: return pick_g<256>(g, merge);
  }
  return nullptr;
}

}  // namespace

size_t attn_work_floats(int batch, int hq, int hd, int max_splits) {
  return static_cast<size_t>(batch) * hq * max_splits * (hd + 2);
}

void launch_attn(const AttnLaunch &L, hipStream_t s) {
  XE_REQUIRE(L.batch > 0 && L.hq > 0 && L.hkv > 0 && L.hq % L.hkv == 0, "attn: bad heads");
  XE_REQUIRE(L.max_ctx > 0, "attn: max_ctx must be > 0");
  XE_REQUIRE(L.max_splits >= 1 && L.max_splits <= 256, "attn: max_splits must be 1..256");
  XE_REQUIRE(L.work, "attn: workspace missing");
  const int g = L.hq / L.hkv;
  AttnFn fn = pick(L.hd, g, false);
  AttnFn merge = pick(L.hd, g, true);
  XE_REQUIRE(fn && merge, "attn: unsupported head_dim / GQA group (hd 64/128/256, group 1/2/4/8)");
  XE_REQUIRE(!L.rope_cos || (L.rope_sin && L.pos), "attn: RoPE needs sin table and positions");
  XE_REQUIRE(!L.k_new || (L.v_new && (L.pos || L.lens || L.fixed_len)), "attn: append needs v_new");
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
  hipLaunchKernelGGL(fn, dim3(L.max_splits, L.hkv, L.batch), dim3(kThreads), 0, s, p);
  XE_HIP(hipGetLastError());
  if (L.max_splits > 1) {
    const int blocks = (g * L.hd + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(merge, dim3(blocks, L.hkv, L.batch), dim3(kThreads), 0, s, p);
    XE_HIP(hipGetLastError());
  }
}

}  // namespace xe
