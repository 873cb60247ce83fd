// ll_kernel.h -- the low-latency persistent decode step kernel (see ll_dev.h
// for the exchange protocol and the roles).  One launch runs n_steps tokens
// for nb <= 4 streams.
#pragma once

#include "ll_dev.h"
#include "step_dev.h"

namespace xe {
namespace ll {

// residual[b] = dequant(E[tok[b]]) (+ P[pos[b] + pos_off]) (* mul); the same
// arithmetic as sdev::embed_block.
__device__ __forceinline__ void embed(const StepParams &sp, const int *tok, const int *pos, float *xr) {
  const int D = sp.d;
  for (int t = threadIdx.x; t < sp.nb * D; t += kT) {
    const int b = t / D, j = t % D;
    int tk = lptr(tok)[b];
    tk = tk < 0 ? 0 : (tk >= sp.vocab ? sp.vocab - 1 : tk);
    int prow = lptr(pos)[b] + sp.pos_off;
    prow = prow < 0 ? 0 : (prow >= sp.pos_rows ? sp.pos_rows - 1 : prow);
    const size_t i = static_cast<size_t>(tk) * D + j;
    float v;
    if (sp.emb_exps)
      v = ldexpf(static_cast<float>(gptr(static_cast<const int8_t *>(sp.emb))[i]),
                 static_cast<int>(gptr(sp.emb_exps)[i / 8]) - 133);
    else if (sp.emb_scale)
      v = static_cast<float>(gptr(static_cast<const int8_t *>(sp.emb))[i]) * gptr(sp.emb_scale)[tk];
    else
      v = __uint_as_float(static_cast<uint32_t>(gptr(static_cast<const uint16_t *>(sp.emb))[i]) << 16);
    if (sp.pos_emb) v = v + gptr(sp.pos_emb)[static_cast<size_t>(prow) * D + j];
    if (sp.use_mul) v = v * sp.emb_mul;
    lptr(xr)[t] = v;
  }
}

// The lm-head slice (its own function: its streaming loop needs a different
// register budget from the per-layer phases).  Arguments by value: a
// reference to the kernel-argument block or to a caller's private struct would
// reach the callee as a generic pointer (flat loads).
struct HeadArgs {
  const void *w;
  const float *scale;
  const uint8_t *exps;
  const float *gamma, *beta;
  float *logits;
  int vocab, d, lpr, rpl, norm, last_max;
  float eps;
};
struct HeadOut {
  ArgBest best;
  int ok;
};

template <int WT, int NB>
__device__ __noinline__ HeadOut head_gemv(const HeadArgs h, int nb, int r0, int r1, float *xr, float *xin,
                                          float *red, float *nw, unsigned ep, const Ctl c) {
  GemvD hg{};
  hg.w = h.w;
  hg.scale = h.scale;
  hg.exps = h.exps;
  hg.m = h.vocab;
  hg.k = h.d;
  hg.lpr = h.lpr;
  hg.rpl = h.rpl;
  HeadOut o;
#pragma unroll
  for (int b = 0; b < kMaxNB; b++) {
    o.best.v[b] = -INFINITY;
    o.best.i[b] = -1;
  }
  pre_w(h.gamma, h.d, nw);
  pre_w(h.beta, h.d, nw + nw_floats(h.d));
  auto prep = [&]() -> bool {
    nw_ready();
    norm_rows(xr, nb, h.d, h.norm, h.eps, xin, red, nw);
    return true;
  };
  if (head_one_round<WT>(h.d, h.lpr))
    o.ok = head_rows<WT, NB>(hg, nb, r0, r1, xin, prep, h.logits, h.vocab, h.last_max, o.best) ? 1 : 0;
  else
    o.ok = gemv_any<WT, NB, true>(hg, nb, r0, r1, xin, ep, prep, h.logits, h.vocab, h.last_max, o.best, c, NoSub{}) ? 1 : 0;
  return o;
}

// One role's step loop (IS_A: the attention side, else the FFN side),
// compiled once per role: each copy holds only its role's phase kinds (the
// attention side: folds, GEMVs, attention, merge and the key/value stage; the
// FFN side: folds, GEMVs, the FFN-output partials and their reduction), so
// neither carries the other's live state through the register allocation
// (one loop for both: b = 1 1 186 against 1 228 tok/s).  A phase kind the
// plan gives the wrong role stops the launch (status 3).
// KV8: the plan has int8 cross K / V (its own instantiation, so the bf16
// kernels keep their register allocation).
template <int WT, int NB, int HD, int G, bool KV8, bool IS_A>
__device__ __forceinline__ void step_role(const StepParams &sp, float4 *lds4, float *red, int &bad, int *s_tok,
                                          int *s_pos, int *s_done, float (*s_bv)[kMaxNB], int (*s_bi)[kMaxNB]) {
  float *lds = reinterpret_cast<float *>(lds4);
  const int nb = sp.nb, D = sp.d;
  const int grid = static_cast<int>(gridDim.x);
  constexpr bool is_a = IS_A;
  // the role's LDS layout (floats; every part 16-byte aligned)
  const int kin = is_a ? sp.kin_a : sp.kin_f, stage_floats = is_a ? sp.stage_a : sp.stage_f;
  const int nph = is_a ? sp.n_a : sp.n_f;
  const XE_CONST Phase *ph = cptr(is_a ? sp.ph_a : sp.ph_f);
  float *xr = lds;                                     // residual copy [nb][D]
  float *xin = xr + static_cast<size_t>(NB) * D;       // GEMV / attention input [nb][kin]
  float *scr = xin + static_cast<size_t>(NB) * kin;    // scratch
  float *stage = scr + ((sp.scratch + 3) & ~3);       // staged weight slices
  float *kvs = stage + stage_floats;                   // key/value stage (attention side)
  uint64_t *tlds = reinterpret_cast<uint64_t *>(kvs + (is_a ? sp.kv_floats : 0));  // trace marks (traced launches)
  const int n_a = (grid + kRoleStride - 1) / kRoleStride;
  const int rank = is_a ? static_cast<int>(blockIdx.x) / kRoleStride
                        : static_cast<int>(blockIdx.x) - static_cast<int>(blockIdx.x) / kRoleStride - 1;
  const int nranks = is_a ? n_a : grid - n_a;
  if (threadIdx.x == 0) bad = 0;
  if (stage_floats > 0 && threadIdx.x < kStageZero / 4) stage[threadIdx.x] = 0.f;  // never copied over
  if (sp.trace)  // slots a workgroup never marks read as 0
    for (int t = threadIdx.x; t < sp.trace_slots; t += kT) lptr(tlds)[t] = 0;
  if (threadIdx.x < nb) {
    const int b = threadIdx.x;
    s_tok[b] = (sp.forced && sp.n_forced > 0) ? gptr(sp.forced)[b] : gptr(sp.tokens)[b];
    s_pos[b] = gptr(sp.pos)[b];
    s_done[b] = sp.stop >= 0 ? gptr(sp.done)[b] : 0;
  }
  __syncthreads();
  const Ctl c{sp.status, sp.limit, &bad};
  const int tslots = sp.n_a + sp.n_f;
  auto mark = [&](int step, int slot) {
    if (sp.trace && step == 0 && threadIdx.x == 0) lptr(tlds)[slot] = wall_clock64();
  };
  // input-ready time of phase i (second block of trace slots)
  auto mark_ready = [&](int step, int i) { mark(step, tslots + 4 + (is_a ? 0 : sp.n_a) + i); };
  mark(0, tslots + 3);
  embed(sp, s_tok, s_pos, xr);
  __syncthreads();
  ArgBest none;

  for (int step = 0; step < sp.n_steps; step++) {
    const unsigned ep = sp.ep0 + static_cast<unsigned>(step);
    bool ok = true;
    for (int i = 0; i < nph && ok; i++) {
      const int kind = ph[i].kind, issue = ph[i].issue, kv_issue = ph[i].kv_issue;
      if (issue >= 0 || kv_issue >= 0) lds_barrier();  // the stages' previous readers are done
      if (issue >= 0) {  // a later phase's weight slice into the stage
        if (!IS_A && ph[issue].kind == LK_DPART) {
          if constexpr (!IS_A) {
            const XE_CONST DpartD &sd = ph[issue].u.dpart;
            int k0, k1;
            dpart_slice(sd, rank, nranks, k0, k1);
            dpart_stage_issue<WT>(sd, k0, k1, stage);
          }
        } else {
          const XE_CONST GemvD &sg = ph[issue].u.gemv;
          const int ulog = (sg.act == ACT_GEGLU_TANH ? 1 : 0) + (sg.out_lds ? 2 : 0);
          int s0, s1;
          rank_rows(sg.m >> ulog, rank, nranks, s0, s1);
          stage_issue<WT>(sg, s0 << ulog, s1 << ulog, stage);
        }
      }
      if constexpr (IS_A) {
        if (kv_issue >= 0) {  // the next attention block's keys / values into the key/value stage
          const XE_CONST AttnD &ka = ph[kv_issue].u.attn;
          const int split = rank % ka.max_splits, rest = rank / ka.max_splits;
          const int kvh = rest % ka.hkv, b = rest / ka.hkv;
          if (b < nb) {
            const int len = ka.fixed_len > 0 ? ka.fixed_len : s_pos[b] + 1;
            if (kv_staged(ka, split, len)) kv_stage_issue<HD>(ka, split, kvh, b, len, kvs);
          }
        }
      }
      switch (kind) {
        case LK_FOLD: {
          const XE_CONST FoldD &fd = ph[i].u.fold;
          pre_w(fd.post_w, D, scr);
          ok = fold(fd, nb, D, xr, xin, red, ep, c, scr);
          mark_ready(step, i);
          break;
        }
        case LK_GEMV: {
          const XE_CONST GemvD &g = ph[i].u.gemv;
          const XE_CONST FoldD *gf = g.folds;
          // GeGLU rows come in (gate, up) pairs: split on pair boundaries;
          // activations kept for LK_DPART: on multiples of four of them
          const int ulog = (g.act == ACT_GEGLU_TANH ? 1 : 0) + (g.out_lds ? 2 : 0);
          int r0, r1;
          rank_rows(g.m >> ulog, rank, nranks, r0, r1);
          r0 <<= ulog;
          r1 <<= ulog;
          auto prep = [&]() -> bool {
            bool r = true;
            // the last fold and an RMS norm share one reduction
            const bool fuse = !g.in_vec && g.nfold > 0 && gf[g.nfold - 1].post_w &&
                              (g.norm == XE_NORM_RMS1P || g.norm == XE_NORM_RMS);
            const int nplain = fuse ? g.nfold - 1 : g.nfold;
            // the gains of every fold and of the norm go to LDS before the
            // first poll: fold f's post gain in region f, then gamma (and
            // beta) (regions of nw_floats(D) floats in the scratch area)
            const int nwf = nw_floats(D);
            for (int f = 0; f < g.nfold; f++) pre_w(gf[f].post_w, D, scr + f * nwf);
            if (!g.in_vec) {
              pre_w(g.gamma, D, scr + g.nfold * nwf);
              if (!fuse) pre_w(g.beta, D, scr + (g.nfold + 1) * nwf);
            }
            for (int f = 0; f < nplain && r; f++) r = fold(gf[f], nb, D, xr, xin, red, ep, c, scr + f * nwf);
            if (r && fuse)
              r = fold_rms(gf[g.nfold - 1], nb, D, xr, xin, red, g.eps, g.norm == XE_NORM_RMS1P, ep, c,
                           scr + (g.nfold - 1) * nwf);
            else if (r && g.in_vec) {
              // one round of loads covers the whole input up to kT * 8 pairs
              // (a second round waits for the first to complete)
              if (nb * g.k > kT * 8) r = get<8>(g.in, nb, g.k, xin, xstride(g.k), ep, c, true);
              else r = get(g.in, nb, g.k, xin, xstride(g.k), ep, c, true);
            }
            else if (r) {
              nw_ready();
              norm_rows(xr, nb, g.k, g.norm, g.eps, xin, red, scr + g.nfold * nwf);
            }
            mark_ready(step, i);
            return r;
          };
          auto tsub = [&](int sub) { mark(step, tslots + 4 + sp.n_a + sp.n_f + kSubSlots * ((is_a ? 0 : sp.n_a) + i) + sub); };
          // A staged GEMV's input is an exchange vector and it applies no
          // residual update (plan_stage stages no other), so its wait is the
          // vector's get alone.
          auto prep_in = [&]() -> bool {
            // one round of loads covers the whole input up to kT * 8 pairs
            // (a second round waits for the first to complete)
            const bool r = nb * g.k > kT * 8 ? get<8>(g.in, nb, g.k, xin, xstride(g.k), ep, c, true)
                                             : get(g.in, nb, g.k, xin, xstride(g.k), ep, c, true);
            mark_ready(step, i);
            return r;
          };
          // staged and streamed weights, and the K-split tail (FFN side
          // only), as separate code paths: each holds only its own state
          // (one path for both: b = 1 1 231 against 1 255 tok/s).  K-segment
          // sums go to the scratch area (its norm gains are read by then).
          if (g.staged)
            ok = gemv_rows<WT, NB, false, XE_CONST GemvD, decltype(prep_in), decltype(tsub), 1, !IS_A>(
                g, nb, r0, r1, xin, ep, prep_in, nullptr, 0, 0, none, tsub, stage, true, scr, xin + g.out_lds, kin);
          else
            ok = gemv_rows<WT, NB, false, XE_CONST GemvD, decltype(prep), decltype(tsub), 0, !IS_A>(
                g, nb, r0, r1, xin, ep, prep, nullptr, 0, 0, none, tsub, stage, false, scr, xin + g.out_lds, kin);
          break;
        }
        case LK_ATTN: {
          if constexpr (IS_A) {
            const XE_CONST AttnD &a = ph[i].u.attn;
            // the first block's K/V loads overlap the wait for q (prep runs once)
            bool need_q = true;
            const int nblk = a.max_splits * a.hkv * nb;
            for (int vb = rank; vb < nblk && ok; vb += nranks) {
              const int split = vb % a.max_splits, rest = vb / a.max_splits;
              const int kvh = rest % a.hkv, b = rest / a.hkv;
              const int len = a.fixed_len > 0 ? a.fixed_len : s_pos[b] + 1;
              int chunk, nsplits;
              ll_split(len, a.max_splits, HD, chunk, nsplits);
              if (split >= nsplits) continue;
              auto prep = [&]() -> bool {
                if (!need_q) return true;
                need_q = false;
                const bool r = get(a.q, nb, a.qn, xin, a.qn, ep, c);
                mark_ready(step, i);
                return r;
              };
              // sub-stage trace: input ready, q/k staged, keys done
              auto tsub = [&](int sub) { mark(step, tslots + 4 + sp.n_a + sp.n_f + kSubSlots * ((is_a ? 0 : sp.n_a) + i) + sub); };
              // every attention phase of a plan has group G (host checks)
              // this rank's first block may sit in the key/value stage
              const bool staged = vb == rank && kv_staged(a, split, len);
              // int8 cross K / V: Whisper's 64-wide single-query-head groups only
              if constexpr (KV8 && HD == 64 && G == 1) {
                if (a.k_scale)
                  ok = attn_block<HD, G, true>(a, split, kvh, b, len, xin, scr, ep, prep, tsub, kvs, staged);
                else
                  ok = attn_block<HD, G, false>(a, split, kvh, b, len, xin, scr, ep, prep, tsub, kvs, staged);
              } else {
                ok = attn_block<HD, G, false>(a, split, kvh, b, len, xin, scr, ep, prep, tsub, kvs, staged);
              }
            }
          } else {
            wrong_role(c);
            ok = false;
          }
          break;
        }
        case LK_DPART: {  // this rank's share of the FFN output projection, as partials
          if constexpr (!IS_A) {
            const XE_CONST DpartD &dp = ph[i].u.dpart;
            int k0, k1;
            dpart_slice(dp, rank, nranks, k0, k1);
            auto tsub = [&](int sub) { mark(step, tslots + 4 + sp.n_a + sp.n_f + kSubSlots * ((is_a ? 0 : sp.n_a) + i) + sub); };
            // the stage copies (issued by the phase before) have landed in every wave
            __builtin_amdgcn_s_waitcnt(0);
            tsub(0);
            __syncthreads();
            mark_ready(step, i);
            dpart_block<WT, NB>(dp, nb, k1 - k0, xin + dp.act_off, kin, stage, scr, rank, ep, tsub);
          } else {
            wrong_role(c);
            ok = false;
          }
          break;
        }
        case LK_REDUCE: {  // the partials summed for this rank's outputs
          if constexpr (!IS_A) {
            const XE_CONST ReduceD &rd = ph[i].u.reduce;
            int r0, r1;
            rank_rows(rd.d, rank, nranks, r0, r1);
            auto tsub = [&](int sub) { mark(step, tslots + 4 + sp.n_a + sp.n_f + kSubSlots * ((is_a ? 0 : sp.n_a) + i) + sub); };
            mark_ready(step, i);
            ok = reduce_block<NB>(rd, nb, r0, r1, scr, ep, c, tsub);
          } else {
            wrong_role(c);
            ok = false;
          }
          break;
        }
        case LK_MERGE: {
          if constexpr (IS_A) {
            const XE_CONST MergeD &mg = ph[i].u.merge;
            const int per_head = mg.hd / kDM;
            const int nblk = nb * mg.hq * per_head;
            for (int vb = rank; vb < nblk && ok; vb += nranks) {
              const int e0 = (vb % per_head) * kDM, rest = vb / per_head;
              const int h = rest % mg.hq, b = rest / mg.hq;
              const int len = mg.fixed_len > 0 ? mg.fixed_len : s_pos[b] + 1;
              ok = merge_block(mg, b, h, e0, len, scr, ep, c);
            }
          } else {
            wrong_role(c);
            ok = false;
          }
          break;
        }
      }
      mark(step, (is_a ? 0 : sp.n_a) + i);
    }
    if (!ok) break;

    // ---- lm-head slice of this workgroup + its argmax partial ----
    ArgBest best;
#pragma unroll
    for (int b = 0; b < kMaxNB; b++) {
      best.v[b] = -INFINITY;
      best.i[b] = -1;
    }
    {
      int r0, r1;
      rank_rows(sp.vocab, static_cast<int>(blockIdx.x), grid, r0, r1);
      const HeadArgs ha{sp.emb, sp.emb_scale, sp.emb_exps, sp.head_gamma, sp.head_beta, sp.logits,
                        sp.vocab, sp.d, sp.head_lpr, sp.head_rpl, sp.head_norm, sp.last_max, sp.head_eps};
      const HeadOut ho = head_gemv<WT, NB>(ha, nb, r0, r1, xr, xin, red, scr, ep, c);
      ok = ho.ok != 0;
      best = ho.best;
    }
    if (!ok) break;
    mark(step, tslots);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int b = 0; b < NB; b++) {
      float v = best.v[b];
      int idx = best.i[b];
      wave_argbest(v, idx, sp.last_max);
      if (lane == 0) {
        s_bv[wave][b] = v;
        s_bi[wave][b] = idx;
      }
    }
    // every store of the step (the KV-cache rows above all, which carry no
    // epoch) has completed before this workgroup's argmax partial is
    // published: agent-scope (sc1) stores are visible to every XCD once
    // complete, so a wait for completion suffices (no L2 write-back)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int parity = static_cast<int>(ep & 1u);
    const Vec argv{sp.arg.p + static_cast<size_t>(parity) * nb * sp.arg.ld, sp.arg.ld, 0};
    if (threadIdx.x < nb) {
      const int b = threadIdx.x;
      float v = -INFINITY;
      int idx = -1;
      for (int w = 0; w < kW; w++)
        if (s_bi[w][b] >= 0 && sdev::better(s_bv[w][b], s_bi[w][b], v, idx, sp.last_max)) {
          v = s_bv[w][b];
          idx = s_bi[w][b];
        }
      put(argv, b, 2 * static_cast<int>(blockIdx.x), v, ep);
      put(argv, b, 2 * static_cast<int>(blockIdx.x) + 1, __int_as_float(idx), ep);
    }
    // ---- every workgroup: the same argmax over all partials ----
    ok = get(argv, nb, 2 * grid, scr, 2 * grid, ep + sp.stall, c);
    if (!ok) break;
    mark(step, tslots + 1);
#pragma unroll
    for (int b = 0; b < NB; b++) {
      float v = -INFINITY;
      int idx = -1;
      if (b < nb)
        for (int w = threadIdx.x; w < grid; w += kT) {
          const float pv = lptr(scr)[b * 2 * grid + 2 * w];
          const int pi = __float_as_int(lptr(scr)[b * 2 * grid + 2 * w + 1]);
          if (pi >= 0 && sdev::better(pv, pi, v, idx, sp.last_max)) {
            v = pv;
            idx = pi;
          }
        }
      wave_argbest(v, idx, sp.last_max);
      if (lane == 0) {
        s_bv[wave][b] = v;
        s_bi[wave][b] = idx;
      }
    }
    __syncthreads();
    if (threadIdx.x < nb) {
      const int b = threadIdx.x;
      float v = -INFINITY;
      int idx = -1;
      for (int w = 0; w < kW; w++)
        if (s_bi[w][b] >= 0 && sdev::better(s_bv[w][b], s_bi[w][b], v, idx, sp.last_max)) {
          v = s_bv[w][b];
          idx = s_bi[w][b];
        }
      if (idx < 0) idx = 0;
      const int ps = s_pos[b];
      // a forced (prompt) step's argmax is not a generated token
      const bool gen = !(sp.forced && step + 1 < sp.n_forced);
      int nxt = gen ? idx : gptr(sp.forced)[(step + 1) * nb + b];
      if (gen && sp.stop >= 0 && (s_done[b] != 0 || idx == sp.stop)) {
        s_done[b] = 1;
        nxt = sp.stop;
      }
      if (blockIdx.x == 0) {
        if (ps >= 0 && ps < sp.hist_stride) gptr_w(sp.hist)[static_cast<size_t>(b) * sp.hist_stride + ps] = idx;
        gptr_w(sp.next)[b] = idx;
        gptr_w(sp.tokens)[b] = nxt;
        gptr_w(sp.pos)[b] = ps + 1;
        if (sp.stop >= 0) gptr_w(sp.done)[b] = s_done[b];
      }
      s_tok[b] = nxt;
      s_pos[b] = ps + 1;
    }
    __syncthreads();
    if (sp.stop >= 0) {  // every workgroup holds the same flags: all leave at the same step
      bool all = true;
      for (int b = 0; b < nb; b++) all = all && s_done[b] != 0;
      if (all) break;
    }
    embed(sp, s_tok, s_pos, xr);
    __syncthreads();
    mark(step, tslots + 2);
    if (sp.trace && step == 0) {
      __syncthreads();
      for (int t = threadIdx.x; t < sp.trace_slots; t += kT)
        gptr_w(sp.trace)[static_cast<size_t>(t) * grid + blockIdx.x] = lptr(tlds)[t];
    }
  }
}

template <int WT, int NB, int HD, int G, bool KV8>
__global__ __launch_bounds__(kT) void ll_step_kernel(StepParams sp) {
  extern __shared__ float4 lds4[];
  __shared__ float red[2 * 4 * gdev::kMaxWaves];
  __shared__ int bad;
  __shared__ int s_tok[kMaxNB], s_pos[kMaxNB], s_done[kMaxNB];
  __shared__ float s_bv[kW][kMaxNB];
  __shared__ int s_bi[kW][kMaxNB];
  if (blockIdx.x % kRoleStride == 0)
    step_role<WT, NB, HD, G, KV8, true>(sp, lds4, red, bad, s_tok, s_pos, s_done, s_bv, s_bi);
  else
    step_role<WT, NB, HD, G, KV8, false>(sp, lds4, red, bad, s_tok, s_pos, s_done, s_bv, s_bi);
}

using StepFn = void (*)(StepParams);

// int8 cross K / V (kv8) is instantiated for int8 weights (the fused decode
// ELF's combination); other weight types with it run the phase kernels.
template <int WT, int NB>
StepFn pick_head(int hd, int g, bool kv8) {
  if (hd == 64 && g == 1) {
    if constexpr (WT == XE_I8)
      if (kv8) return ll_step_kernel<WT, NB, 64, 1, true>;
    return kv8 ? nullptr : ll_step_kernel<WT, NB, 64, 1, false>;
  }
  if (hd == 256 && g == 4 && !kv8) return ll_step_kernel<WT, NB, 256, 4, false>;
  return nullptr;
}

template <int WT>
StepFn pick_nb(int nb, int hd, int g, bool kv8) {
  switch (nb) {
    case 1: return pick_head<WT, 1>(hd, g, kv8);
    case 2: return pick_head<WT, 2>(hd, g, kv8);
    case 4: return pick_head<WT, 4>(hd, g, kv8);
  }
  return nullptr;
}

// one translation unit per weight dtype (ll_i8.hip, ll_bf16.hip, ll_bfp16.hip)
StepFn pick_ll_i8(int nb, int hd, int g, bool kv8);
StepFn pick_ll_bf16(int nb, int hd, int g, bool kv8);
StepFn pick_ll_bfp16(int nb, int hd, int g, bool kv8);

}  // namespace ll
}  // namespace xe
