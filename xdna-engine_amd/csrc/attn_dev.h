// attn_dev.h -- device side of single-query attention over a bf16 KV cache
// (split-K flash decode).
//
// Replaces the reference's mha_decode (route_b_kernels/mha_decode/
// mha_decode.cc:90-175: online softmax per key over streamed K/V tiles with a
// runtime key count) and its host driver CtxDecode::attn
// (rust/npu-asr/src/ctx_decode.rs:468-555), generalised to GQA, head_dim
// 64/128/256, per-stream lengths and contexts far beyond the reference's 448.
// The arithmetic target is attend_one (whisper_decoder.rs:242-278): scores
// (q.k) * scale in fp32, softmax, p-weighted sum of V.
//
// One "split block" takes one contiguous key range of one (stream, kv head)
// and all G = hq/hkv query heads that share it, so the K/V bytes of a GQA
// group are read once:
//   * L = hd/8 lanes hold one key (16 B of bf16 each); a wave reads 64/L
//     consecutive keys per load: whole 128-byte lines.
//   * Each lane group keeps an online-softmax state (m, l, acc) per query head
//     in registers, updated once per block of UK keys (log2 domain, exp2).
//   * Lane groups merge by xor-shuffles, waves through LDS; the block writes
//     (m, l, acc) to the workspace (or the output when one split covers the
//     whole length).
// A "merge block" finishes 256 of the G*hd outputs of one (stream, kv head)
// from the split partials, as a launch of its own (a caller's workspace
// without counters).  With arrival counters (AttnParams::cnt) the split
// kernel merges in place instead: each split block stores
// its partial with sc1 stores (past the XCD's own L2), waits for them, counts
// itself in the (stream, kv head)'s counter with an agent-scope atomic, and
// the last to arrive reads every partial with sc1 loads and writes the output
// (no device-scope release/acquire fences: those write back and invalidate L2
// on this part and measured ~80 us per launch).
// Fused in front (decode step): the Gemma per-head RMSNorm (1 + w) and RoPE of
// q and the new k, and the bf16 append of the new k/v at position pos, done
// by the block whose range holds pos (the only one that reads it).
// int8 K and/or V (KV8 bit 0 / bit 1; Whisper's per-utterance cross K/V,
// route_b_kernels/decode_fused/gen_decode.py:263-282): 8 int8 of a key a
// lane (8-byte loads); the per-channel K scale multiplies q once
// (scores = sum_d (q[d] s_k[d]) k8[d]), the V scale multiplies the p-weighted
// sums when they are written (out[d] = s_v[d] sum_t p_t v8[t][d]).
#pragma once

#include "gemv_dev.h"

namespace xe {
namespace adev {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMinChunk = 64;  // keys per split at least (amortises per-block setup)
constexpr int kMaxSplits = 256;

using gdev::act_ld;
using gdev::act_st;
using gdev::wave_sum;

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
  const float *k_scale, *v_scale;  // int8 K / V channel scales [hkv * hd], or null (bf16)
  unsigned *cnt;  // [batch * hkv] arrival counters (zero between launches): merge in the
                  // split kernel; null: a merge phase follows
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  // Integer RNE with quiet-NaN, bit-identical to f32_to_bf16_bits
  // (rust/npu-xrt/src/lib.rs:809-817).
  // Branch-free (a select), so unrolled conversions stay one basic block.
  const uint32_t bits = __float_as_uint(x);
  const uint32_t rounded = (bits + 0x00007fffu + ((bits >> 16) & 1u)) >> 16;
  const uint32_t quiet = (bits >> 16) | 0x0040u;
  return static_cast<uint16_t>((bits & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

// Filled length of stream b.  A length outside [1, max_ctx] (a device-side
// length array the host cannot check, or a position past the cache) makes
// the stream's blocks return at once: no K/V row is appended or read past
// the cache, and the stream's output is left as it was.
__device__ __forceinline__ int stream_len(const AttnParams &p, int b) {
  const int len = p.lens ? p.lens[b] : p.pos ? p.pos[b] + 1 : p.fixed_len;
  return len > p.max_ctx ? 0 : len;
}

__host__ __device__ __forceinline__ void split_range(int len, int max_splits, int &chunk, int &nsplits) {
  int per = (len + max_splits - 1) / max_splits;
  per = (per + kMinChunk - 1) / kMinChunk * kMinChunk;
  chunk = per < kMinChunk ? kMinChunk : per;
  nsplits = (len + chunk - 1) / chunk;
}

// LDS floats a split block / merge block needs.
__host__ __device__ constexpr size_t attn_lds_floats(int hd, int g) {
  return static_cast<size_t>(g) * hd + static_cast<size_t>(kWaves) * g * (hd + 2);
}
__host__ __device__ constexpr size_t merge_lds_floats() {
  return static_cast<size_t>(4) * kMaxSplits + 4;
}

// Per-head RMSNorm (1+w) and RoPE on one head vector held by one wave:
// lane j (< hd/2) owns elements (j, j + hd/2) for j = lane, lane + 64, ...
template <int HD, bool COH>
__device__ __forceinline__ void head_transform(const AttnParams &p, const float *src, float *dst,
                               const float *norm_w, int posi) {
  constexpr int HALF = HD / 2;
  constexpr int PER = (HALF + 63) / 64;
  const int lane = threadIdx.x & 63;
  float a[PER], c[PER];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int j = lane + 64 * i;
    a[i] = j < HALF ? act_ld<COH>(src, j) : 0.f;
    c[i] = j < HALF ? act_ld<COH>(src, j + HALF) : 0.f;
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

// A lane's eight elements of one key row, loaded raw (16 bytes of bf16 or 8
// of int8) and converted at use, so the loads of a block stay in flight
// while earlier keys compute.  NT: rows each stream reads once a step
// (per-stream caches) come in with nontemporal loads (a 168 MB stream over
// 256 workgroups: 24.9 against 27.9 us with plain loads; b = 64 decode
// +1.3 %); rows every stream reads (a cross-attention cache shared by the
// batch) with plain ones, so they stay cached between streams (Whisper-small
// b = 32: 34.8k tok/s against 33.8k with nontemporal loads).
template <bool I8, bool NT = true>
struct Raw8 {
  uint32_t w[I8 ? 2 : 4];
  __device__ __forceinline__ void load(const uint16_t *base, size_t elem) {
    if constexpr (I8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 *src = reinterpret_cast<const u32x2 *>(reinterpret_cast<const int8_t *>(base) + elem);
      u32x2 v;
      if constexpr (NT) v = __builtin_nontemporal_load(src);
      else v = *src;
      w[0] = v.x;
      w[1] = v.y;
    } else {
      const gdev::u32x4 *src = reinterpret_cast<const gdev::u32x4 *>(base + elem);
      gdev::u32x4 v;
      if constexpr (NT) v = __builtin_nontemporal_load(src);
      else v = *src;
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
    }
  }
  __device__ __forceinline__ float get(int e) const {
    if constexpr (I8)
      return static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(static_cast<int>(w[e >> 2]), 8 * (e & 3), 8)));
    else
      return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  }
};

// Phase 1 of a merge, heads [g0, g0 + ng) of one (stream, kv head) (waves
// over heads, lanes over splits): wts[hh][s] = exp2(m_s - M) with M the
// largest m_s, lsum[hh] = sum_s l_s wts[hh][s].  wbase: the partials of the
// (stream, kv head), head g's split s at (g * max_splits + s) * (HD + 2).
template <int HD, bool LDCOH>
__device__ __forceinline__ void merge_weights(const AttnParams &p, const float *wbase, int nsplits, int g0, int ng,
                                              float *wts, float *lsum) {
  constexpr int RS = HD + 2;  // floats of one partial: m, l, acc[HD]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int hh = wave; hh < ng; hh += kWaves) {
    const int row = (g0 + hh) * p.max_splits;
    float ls = 0.f;
    if (nsplits <= 64) {  // one split a lane: m and l in one round trip
      const bool on = lane < nsplits;
      const int src = (row + (on ? lane : 0)) * RS;
      const float ms = act_ld<LDCOH>(wbase, src), lv = act_ld<LDCOH>(wbase, src + 1);
      float mx = on ? ms : -INFINITY;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float f = !on || ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
      if (on) {
        wts[hh * kMaxSplits + lane] = f;
        ls = lv * f;
      }
    } else {
      float mx = -INFINITY;
      for (int sidx = lane; sidx < nsplits; sidx += 64) mx = fmaxf(mx, act_ld<LDCOH>(wbase, (row + sidx) * RS));
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      for (int sidx = lane; sidx < nsplits; sidx += 64) {
        const int src = (row + sidx) * RS;
        const float ms = act_ld<LDCOH>(wbase, src);
        const float f = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
        wts[hh * kMaxSplits + sidx] = f;
        ls += act_ld<LDCOH>(wbase, src + 1) * f;
      }
    }
    ls = wave_sum(ls);
    if (lane == 0) lsum[hh] = ls;
  }
}

// Merges heads [g0, g0 + ng) of (stream b, kv head kvh) from the nsplits
// partials: out = sum_s acc_s w_s / sum_s l_s w_s (even and odd splits summed
// apart, in split order, then added).  A thread takes outputs threadIdx.x +
// j * kThreads, j < NE (ng * HD <= NE * kThreads).  The acc values of splits
// [0, 8) are loaded before phase 1, so with at most 8 splits the merge takes
// one memory round trip.  LDCOH: sc1 loads of the partials; STCOH:
// agent-scope output stores.  lds: ng * (kMaxSplits + 1) floats.
template <int HD, int G, int NE, bool LDCOH, bool STCOH>
__device__ __forceinline__ void merge_heads(const AttnParams &p, int kvh, int b, int nsplits, int g0, int ng,
                                            float *lds) {
  constexpr int RS = HD + 2;
  constexpr int SC = 8;  // splits a thread holds in registers at once
  float *wts = lds;                     // [ng][kMaxSplits]
  float *lsum = lds + ng * kMaxSplits;  // [ng]
  const float *wbase = p.work + (static_cast<size_t>(b) * p.hq + kvh * G) * p.max_splits * RS;
  int src[NE], hw[NE];
  bool ok[NE];
  float at0[NE], at1[NE], v[SC][NE];
#pragma unroll
  for (int j = 0; j < NE; j++) {
    const int t = threadIdx.x + j * kThreads;
    ok[j] = t < ng * HD;
    const int hh = ok[j] ? t / HD : 0, e = t % HD;
    src[j] = (g0 + hh) * p.max_splits * RS + 2 + e;
    hw[j] = hh * kMaxSplits;
    at0[j] = 0.f;
    at1[j] = 0.f;
  }
  auto load = [&](int s0) {
#pragma unroll
    for (int u = 0; u < SC; u++)
#pragma unroll
      for (int j = 0; j < NE; j++)
        v[u][j] = ok[j] && s0 + u < nsplits ? act_ld<LDCOH>(wbase, src[j] + (s0 + u) * RS) : 0.f;
  };
  load(0);
  merge_weights<HD, LDCOH>(p, wbase, nsplits, g0, ng, wts, lsum);
  __syncthreads();
  for (int s0 = 0; s0 < nsplits; s0 += SC) {
    if (s0) load(s0);
#pragma unroll
    for (int u = 0; u < SC; u++) {
      if (s0 + u >= nsplits) break;
#pragma unroll
      for (int j = 0; j < NE; j++) {
        if (!ok[j]) continue;
        if (u & 1) at1[j] += v[u][j] * wts[hw[j] + s0 + u];
        else at0[j] += v[u][j] * wts[hw[j] + s0 + u];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NE; j++) {
    if (!ok[j]) continue;
    const int t = threadIdx.x + j * kThreads, hh = t / HD, e = t % HD;
    const float at = at0[j] + at1[j];
    const float o = p.div_norm ? at / lsum[hh] : at * (1.0f / lsum[hh]);
    act_st<STCOH>(p.out + static_cast<size_t>(b) * p.out_stride + (kvh * G + g0 + hh) * HD + e, o);
  }
}

// One split block: keys [split*chunk, ...) of (stream b, kv head kvh).
// NT: the key / value loads are nontemporal (Raw8).
template <int HD, int G, bool COH, int KV8 = 0, bool NT = true>
__device__ __forceinline__ void attn_split_block(const AttnParams &p, int split, int kvh, int b, float *lds) {
  constexpr bool K8 = (KV8 & 1) != 0, V8 = (KV8 & 2) != 0;
  constexpr int EPL = 8;       // elements per lane per key (16 B of bf16, 8 B of int8)
  constexpr int L = HD / EPL;  // lanes per key
  constexpr int kLog2L = L == 8 ? 3 : L == 16 ? 4 : L == 32 ? 5 : 6;
  static_assert((1 << kLog2L) == L, "lanes per key: 8, 16, 32 or 64");
  constexpr int KPW = 64 / L;  // keys per wave per load
  constexpr int UK = 4;        // keys per lane group per block update
  constexpr int STEP = kWaves * KPW;
  float(*qs)[HD] = reinterpret_cast<float(*)[HD]>(lds);
  float(*red)[G][HD + 2] = reinterpret_cast<float(*)[G][HD + 2]>(lds + G * HD);

  const int len = stream_len(p, b);
  if (len <= 0) return;
  int chunk, nsplits;
  split_range(len, p.max_splits, chunk, nsplits);
  if (split >= nsplits) return;
  const int s0 = split * chunk;
  const int s1 = min(len, s0 + chunk);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int posi = len - 1;

  // element offsets (bytes for int8, uint16 units for bf16 through load8)
  const size_t kvoff = p.kv_bstride * b + static_cast<size_t>(kvh) * p.max_ctx * HD;
  uint16_t *kbase = p.kc + (K8 ? 0 : kvoff);
  uint16_t *vbase = p.vc + (V8 ? 0 : kvoff);
  const size_t kel = K8 ? kvoff : 0, vel = V8 ? kvoff : 0;

  const int kg = lane / L, kl = lane % L;
  const int base0 = s0 + wave * KPW + kg;
  const bool appender = !K8 && !V8 && p.k_new && split == nsplits - 1;
  // UK keys' K and V rows from `base` (keys past the range read key s0)
  auto load_block = [&](int base, Raw8<K8, NT> (&kv)[UK], Raw8<V8, NT> (&vv)[UK], bool (&ok)[UK]) {
#pragma unroll
    for (int u = 0; u < UK; u++) {
      const int key = base + u * STEP;
      ok[u] = key < s1;
      const int kk = ok[u] ? key : s0;
      kv[u].load(kbase, kel + static_cast<size_t>(kk) * HD + kl * EPL);
      vv[u].load(vbase, vel + static_cast<size_t>(kk) * HD + kl * EPL);
    }
  };
  // the first block's loads go out before the head transforms, so their HBM
  // latency overlaps the prologue (not in the appender's block: it reads
  // back the row it appends)
  Raw8<K8, NT> kv0[UK];
  Raw8<V8, NT> vv0[UK];
  bool ok0[UK];
  if (!appender) load_block(base0, kv0, vv0, ok0);

  // ---- q heads of this group (norm + rope), new k/v append ----
  for (int g = wave; g < G; g += kWaves) {
    const float *src = p.q + static_cast<size_t>(b) * p.q_stride + (kvh * G + g) * HD;
    head_transform<HD, COH>(p, src, qs[g], p.q_norm_w, posi);
  }
  if (appender && wave == 0) {
    const float *ksrc = p.k_new + static_cast<size_t>(b) * p.kv_new_stride + kvh * HD;
    const float *vsrc = p.v_new + static_cast<size_t>(b) * p.kv_new_stride + kvh * HD;
    float *kt = red[0][0];  // scratch: transformed k
    head_transform<HD, COH>(p, ksrc, kt, p.k_norm_w, posi);
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < HD; j += 64) {
      kbase[static_cast<size_t>(posi) * HD + j] = f32_to_bf16_rne(kt[j]);
      vbase[static_cast<size_t>(posi) * HD + j] = f32_to_bf16_rne(act_ld<COH>(vsrc, j));
    }
  }
  __syncthreads();  // the appended row is read back by this block only

  // ---- main loop: online softmax per lane group ----
  float qr[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int e = 0; e < EPL; e++)
      qr[g][e] = K8 ? qs[g][kl * EPL + e] * p.k_scale[kvh * HD + kl * EPL + e] : qs[g][kl * EPL + e];
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[g][e] = 0.f;
  }
  const float sc2 = p.scale * kLog2e;

  // one block of UK keys per lane group: scores, online softmax, P.V
  auto block = [&](const Raw8<K8, NT>(&kv)[UK], const Raw8<V8, NT>(&vv)[UK], const bool(&ok)[UK]) {
    // the block's UK x G partial dot products, then their sums over the L
    // lanes of each key, level by level through DPP and permlane swaps (no
    // LDS crossbar round trips)
    float sd[UK * G];
#pragma unroll
    for (int u = 0; u < UK; u++) {
      float kf[EPL];
#pragma unroll
      for (int e = 0; e < EPL; e++) kf[e] = kv[u].get(e);
#pragma unroll
      for (int g = 0; g < G; g++) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) d = __builtin_fmaf(qr[g][e], kf[e], d);
        sd[u * G + g] = d;
      }
    }
    gdev::group_sums<UK * G>(sd, kLog2L);
    float s[UK][G];
#pragma unroll
    for (int u = 0; u < UK; u++)
#pragma unroll
      for (int g = 0; g < G; g++) s[u][g] = sd[u * G + g] * sc2;
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
      for (int u = 0; u < UK; u++)
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = __builtin_fmaf(pu[u], vv[u].get(e), acc[g][e]);
    }
  };
  // two blocks in flight: the next block's loads go out before this block's
  // arithmetic (keys past the range read key s0 and are masked)
  constexpr int BS = STEP * UK;
  Raw8<K8, NT> kb[UK];
  Raw8<V8, NT> vb[UK];
  bool ob[UK];
  if (appender) load_block(base0, kv0, vv0, ok0);
  for (int base = base0; base < s1; base += 2 * BS) {
    load_block(base + BS, kb, vb, ob);
    block(kv0, vv0, ok0);
    if (base + BS >= s1) break;
    load_block(base + 2 * BS, kv0, vv0, ok0);
    block(kb, vb, ob);
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
  // merge in place (standalone kernel with arrival counters): the partials
  // go out with sc1 stores
  const bool fuse = !COH && p.cnt && !single;
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
    if (V8) at = at * p.v_scale[kvh * HD + e];
    if (single) {
      const float o = p.div_norm ? at / lt : at * (1.0f / lt);
      act_st<COH>(p.out + static_cast<size_t>(b) * p.out_stride + (kvh * G + g) * HD + e, o);
    } else {
      float *dst = wbase + (static_cast<size_t>(g) * p.max_splits + split) * (HD + 2);
      if (COH || fuse) {
        act_st<true>(dst + 2 + e, at);
        if (e == 0) {
          act_st<true>(dst, mx);
          act_st<true>(dst + 1, lt);
        }
      } else {
        act_st<false>(dst + 2 + e, at);
        if (e == 0) {
          act_st<false>(dst, mx);
          act_st<false>(dst + 1, lt);
        }
      }
    }
  }
  if constexpr (!COH) {
    if (fuse) {
      // arrival: this wave's partial stores have completed before the count
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      unsigned *cnt = p.cnt + static_cast<size_t>(b) * p.hkv + kvh;
      int *flag = reinterpret_cast<int *>(lds);
      if (threadIdx.x == 0)
        flag[0] = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  static_cast<unsigned>(nsplits - 1);
      __syncthreads();
      const bool last = flag[0] != 0;
      __syncthreads();  // the flag is read before merge_heads reuses the LDS
      if (last) {
        merge_heads<HD, G, (G * HD + kThreads - 1) / kThreads, true, false>(p, kvh, b, nsplits, 0, G, lds);
        if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __syncthreads();  // LDS is reused by the caller's next block
}

// Merge block `blk` of (stream b, kv head kvh): outputs blk*256 .. +256 of the
// G*HD, i.e. heads [blk * HPB, +HPB) with HPB = 256 / HD.
template <int HD, int G, bool COH>
__device__ __forceinline__ void attn_merge_block(const AttnParams &p, int blk, int kvh, int b, float *lds) {
  constexpr int HPB = kThreads >= HD ? kThreads / HD : 1;  // heads per block
  const int len = stream_len(p, b);
  if (len <= 0) return;
  int chunk, nsplits;
  split_range(len, p.max_splits, chunk, nsplits);
  if (nsplits == 1) return;  // the split block wrote the output
  const int g0 = blk * HPB;
  if (g0 >= G) return;
  merge_heads<HD, G, 1, COH, COH>(p, kvh, b, nsplits, g0, min(HPB, G - g0), lds);
  __syncthreads();  // LDS is reused by the caller's next block
}

AttnParams to_params(const AttnLaunch &L);

}  // namespace adev
}  // namespace xe
