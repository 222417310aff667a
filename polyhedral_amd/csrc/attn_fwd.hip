// C-ABI entry of the attention forward: argument checks, then dispatch to the
// (dtype, D, waves) instantiation.  Mirrors the checks of the reference entry
// point gpu/triton_attn.py:185-241 (N % BQ, N % A, shapes) and reports them as
// PA_E_INVALID with a message instead of an AssertionError.
#include "attn_kernel.hpp"

namespace pa {
int launch_attn_bf16(const AttnK& a, int D, int NW, hipStream_t s);
int launch_attn_f16(const AttnK& a, int D, int NW, hipStream_t s);
int launch_attn_f32(const AttnK& a, int D, int NW, hipStream_t s);
int launch_attn_wsplit(const AttnK& a, int D, hipStream_t s);
int launch_attn_stream(const AttnK& a, int dtype, hipStream_t s);
int launch_attn_run(const AttnK& a, int groups, int dtype, bool cooperative, hipStream_t s);
int launch_attn_split_grid(const AttnK& a, int dtype, hipStream_t s);
}  // namespace pa

namespace pa {
// Checks every argument of one launch and fills the kernel arguments (no launch).
static int fill_attn(const pa_attn_args* x, AttnK& a) {
  PA_CHECK_ARG(x != nullptr, "pa_attn_fwd: null args");
  PA_CHECK_ARG(x->q && x->k && x->v && x->o, "pa_attn_fwd: null q/k/v/o");
  PA_CHECK_ARG(x->kv_num, "pa_attn_fwd: null kv_num");
  // an index whose every list is empty has pitch 0 and no list storage
  PA_CHECK_ARG(x->pitch == 0 || (x->kv_idx && x->kv_partial), "pa_attn_fwd: null kv_idx / kv_partial");
  PA_CHECK_ARG(x->D == 64 || x->D == 128, "pa_attn_fwd: D=%d (supported: 64, 128)", x->D);
  PA_CHECK_ARG(x->dtype == PA_F32 || x->dtype == PA_F16 || x->dtype == PA_BF16, "pa_attn_fwd: dtype %d",
               x->dtype);
  PA_CHECK_ARG(x->BH >= 1 && x->N >= 1 && x->N <= (1ll << 30), "pa_attn_fwd: BH=%lld N=%lld",
               (long long)x->BH, (long long)x->N);
  const bool tile_ok = (x->BQ == 16 || x->BQ == 32 || x->BQ == 64 || x->BQ == 128) &&
                       (x->A == 16 || x->A == 32 || x->A == 64 || x->A == 128);
  PA_CHECK_ARG(tile_ok, "pa_attn_fwd: tile %dx%d (BQ, A each in 16, 32, 64, 128)", x->BQ, x->A);
  PA_CHECK_ARG(x->N % x->BQ == 0 && x->N % x->A == 0, "pa_attn_fwd: N=%lld not divisible by BQ=%d, A=%d",
               (long long)x->N, x->BQ, x->A);
  PA_CHECK_ARG(x->pitch >= 0, "pa_attn_fwd: negative pitch");
  PA_CHECK_ARG(x->pitch == 0 || !x->kv_bits_off == !x->kv_bits,
               "pa_attn_fwd: kv_bits_off and kv_bits go together");
  PA_CHECK_ARG(x->residue_s <= 0 ||
                   (x->residue_qlog2 >= 4 && x->residue_qlog2 < 31 &&
                    (int64_t)x->residue_s << x->residue_qlog2 == x->N),
               "pa_attn_fwd: residue_s=%d with N/s = 2^%d does not match N=%lld (N/s >= 16 needed)",
               x->residue_s, x->residue_qlog2, (long long)x->N);
  {
    // a 16-row segment's in-head byte offsets are 32-bit in the kernel
    const int64_t esz0 = x->dtype == PA_F32 ? 4 : 2;
    const int64_t stride = x->residue_s > 0 ? x->residue_s : 1;
    const int64_t rb = (x->k_sn > x->v_sn ? x->k_sn : x->v_sn) * esz0;
    PA_CHECK_ARG(16 * stride * rb < (1ll << 31), "pa_attn_fwd: row stride too large for 32-bit offsets");
  }
  PA_CHECK_ARG(!(x->gather_q || x->scatter_o) || x->mask.perm_q || x->residue_s > 0,
               "pa_attn_fwd: gather_q / scatter_o need mask.perm_q or residue_s");
  PA_CHECK_ARG(!x->gather_kv || x->mask.perm_kv || x->residue_s > 0,
               "pa_attn_fwd: gather_kv needs mask.perm_kv or residue_s");
  PA_CHECK_ARG(!x->prev_o || x->prev_lse, "pa_attn_fwd: prev_o needs prev_lse");
  PA_CHECK_ARG(!x->prev_o || x->prev_dtype == PA_F32 || x->prev_dtype == PA_F16 || x->prev_dtype == PA_BF16,
               "pa_attn_fwd: prev_dtype %d", x->prev_dtype);
  PA_CHECK_ARG(!x->prev_o || x->lse_sb >= x->N, "pa_attn_fwd: lse_sb=%lld < N", (long long)x->lse_sb);
  PA_CHECK_ARG(!x->lse || x->lse_sb >= x->N, "pa_attn_fwd: lse_sb=%lld < N", (long long)x->lse_sb);
  if (int rc = check_mask(&x->mask, x->N)) return rc;
  // 16-B vector access of every row start
  const int esz = x->dtype == PA_F32 ? 4 : 2;
  auto al = [&](const void* p, int64_t sb, int64_t sn) {
    return (reinterpret_cast<uintptr_t>(p) % 16) == 0 && (sb * esz) % 16 == 0 && (sn * esz) % 16 == 0;
  };
  PA_CHECK_ARG(al(x->q, x->q_sb, x->q_sn) && al(x->k, x->k_sb, x->k_sn) && al(x->v, x->v_sb, x->v_sn) &&
                   al(x->o, x->o_sb, x->o_sn),
               "pa_attn_fwd: q/k/v/o rows must be 16-byte aligned");

  a = AttnK{};
  a.q = static_cast<const char*>(x->q);
  a.k = static_cast<const char*>(x->k);
  a.v = static_cast<const char*>(x->v);
  a.o = static_cast<char*>(x->o);
  a.q_sb = x->q_sb; a.q_sn = x->q_sn;
  a.k_sb = x->k_sb; a.k_sn = x->k_sn;
  a.v_sb = x->v_sb; a.v_sn = x->v_sn;
  a.o_sb = x->o_sb; a.o_sn = x->o_sn;
  a.N = (int32_t)x->N;
  a.BQ = x->BQ;
  a.A = x->A;
  a.spt_log2 = x->A == 16 ? 0 : x->A == 32 ? 1 : x->A == 64 ? 2 : 3;
  a.nq = (int32_t)(x->N / x->BQ);
  a.total_wg = (int64_t)a.nq * x->BH;
  a.c = x->scale * 1.4426950408889634f;
  a.kv_idx = x->kv_idx;
  a.kv_num = x->kv_num;
  a.kv_partial = x->kv_partial;
  a.kv_wave_bits = x->kv_wave_bits;
  a.pitch = x->pitch;
  a.kv_bits_off = x->kv_bits_off;
  a.kv_bits = x->kv_bits;
  a.pred = make_pred(x->mask);
  a.gather_q = x->gather_q;
  a.gather_kv = x->gather_kv;
  a.scatter_o = x->scatter_o;
  a.residue_s = x->residue_s > 0 ? x->residue_s : 0;
  a.residue_qlog2 = x->residue_s > 0 ? x->residue_qlog2 : 0;
  a.lse = x->lse;
  a.lse_sb = x->lse_sb;
  a.prev_o = static_cast<const char*>(x->prev_o);
  a.prev_dtype = x->prev_dtype;
  a.prev_sb = x->prev_sb;
  a.prev_sn = x->prev_sn;
  a.prev_lse = x->prev_lse;
  a.qblock_order = x->qblock_order;
  a.steps = x->kv_steps;
  a.steps_pitch = x->steps_pitch;
  a.BH = x->BH;
  a.heads_desc = x->heads_desc != 0;
  a.gather_mult = x->gather_mult > 1 ? x->gather_mult : 1;
  a.gather_scatter = x->gather_scatter != 0;
  a.wsel = static_cast<const char*>(x->wsel);
  a.wsel_sb = x->wsel_sb;
  PA_CHECK_ARG(x->gather_mult <= 1 || (x->wsel && x->wsel_sb >= x->gather_mult),
               "pa_attn_fwd: gather_mult=%d needs wsel [BH, >= gather_mult]", x->gather_mult);
  PA_CHECK_ARG(x->gather_mult <= 1 || !x->kv_steps,
               "pa_attn_fwd: gather_mult > 1 runs on the general kernel (pass no kv_steps)");
  PA_CHECK_ARG(x->gather_mult <= 64, "pa_attn_fwd: gather_mult=%d too large", x->gather_mult);
  PA_CHECK_ARG(a.total_wg <= 0x7fffffffll, "pa_attn_fwd: %lld work-groups exceed the grid limit",
               (long long)a.total_wg);

  a.run_steps = x->run_steps;
  a.run_start = x->run_start;
  a.run_res[0] = a.residue_s;
  a.run_qlog2[0] = a.residue_qlog2;
  a.run_flags[0] = (x->gather_q ? kPieceGatherQ : 0) | (x->gather_kv ? kPieceGatherKV : 0) |
                   (x->scatter_o ? kPieceScatterO : 0) | (x->prev_o ? kPieceMerge : 0);
  if (x->run_groups > 0) {
    // the persistent streaming kernel: asked for by passing a schedule
    PA_CHECK_ARG(x->dtype == PA_BF16 || x->dtype == PA_F16, "pa_attn_fwd: run_groups needs f16 or bf16");
    PA_CHECK_ARG(x->D == 128 && x->BQ == 128 && (x->A == 16 || x->A == 32 || x->A == 64),
                 "pa_attn_fwd: run_groups needs D = 128, BQ = 128, A in 16, 32, 64 (got D=%d, %dx%d)", x->D, x->BQ,
                 x->A);
    PA_CHECK_ARG(x->run_steps && x->run_start, "pa_attn_fwd: run_groups needs run_steps and run_start");
    PA_CHECK_ARG((reinterpret_cast<uintptr_t>(x->run_steps) & 15) == 0, "pa_attn_fwd: run_steps not 16-byte aligned");
    PA_CHECK_ARG(x->pitch == 0 || x->kv_bits, "pa_attn_fwd: run_groups needs the partial-tile bitmaps");
    PA_CHECK_ARG(x->gather_mult <= 1, "pa_attn_fwd: gather_mult > 1 runs on the general kernel");
    PA_CHECK_ARG(!(x->gather_q || x->scatter_o || x->gather_kv) || x->residue_s > 0,
                 "pa_attn_fwd: run_groups gathers and scatters through the closed-form residue basis only");
    PA_CHECK_ARG(x->k_sb == x->N * x->k_sn && x->v_sb == x->N * x->v_sn,
                 "pa_attn_fwd: run_groups needs k and v with batch stride N * row stride");
    const int64_t rb = (x->k_sn > x->v_sn ? x->k_sn : x->v_sn) * 2;
    PA_CHECK_ARG(x->BH * x->N * rb < (1ll << 32), "pa_attn_fwd: BH * N * row bytes too large for run_groups");
  }
  return PA_OK;
}
}  // namespace pa

extern "C" int pa_attn_fwd(const pa_attn_args* x, void* stream) {
  pa::AttnK a;
  if (int rc = pa::fill_attn(x, a)) return rc;
  const int NW = x->BQ >= 32 ? x->BQ / 32 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x->run_groups > 0) return pa::launch_attn_run(a, x->run_groups, x->dtype, false, s);
  if (x->wave_split) {
    // the wave-split kernel: asked for explicitly, so its preconditions are errors
    PA_CHECK_ARG(x->dtype == PA_F32 && (x->D == 64 || x->D == 128),
                 "pa_attn_fwd: wave_split needs float32 with D = 64 or 128");
    PA_CHECK_ARG(x->BQ % 32 == 0 && x->A % 32 == 0, "pa_attn_fwd: wave_split needs BQ and A multiples of 32");
    PA_CHECK_ARG(x->kv_wave_bits || x->pitch == 0, "pa_attn_fwd: wave_split needs kv_wave_bits");
    PA_CHECK_ARG(!x->gather_q && !x->gather_kv && !x->scatter_o && x->residue_s <= 0 && !x->mask.perm_q &&
                     !x->mask.perm_kv,
                 "pa_attn_fwd: wave_split takes no permutation");
    PA_CHECK_ARG(x->gather_mult <= 1 && !x->prev_o && !x->kv_steps,
                 "pa_attn_fwd: wave_split takes no class-B emulation, prev_o or kv_steps");
    PA_CHECK_ARG(x->BH * (x->N / 16) < (1ll << 31), "pa_attn_fwd: wave_split grid too large");
    return pa::launch_attn_wsplit(a, x->D, s);
  }
  if (x->kv_steps) {
    // the streaming kernel: asked for by passing the step descriptors, so its
    // preconditions are errors rather than a silent change of kernel
    PA_CHECK_ARG(x->dtype == PA_BF16 || x->dtype == PA_F16, "pa_attn_fwd: kv_steps needs f16 or bf16");
    PA_CHECK_ARG(x->D == 128 && x->BQ == 128 && (x->A == 16 || x->A == 32 || x->A == 64),
                 "pa_attn_fwd: kv_steps needs D = 128, BQ = 128, A in 16, 32, 64 (got D=%d, %dx%d)", x->D, x->BQ,
                 x->A);
    PA_CHECK_ARG(!x->gather_kv || x->residue_s > 0,
                 "pa_attn_fwd: kv_steps supports gather_kv only through the closed-form residue basis");
    PA_CHECK_ARG(x->pitch == 0 || x->kv_bits, "pa_attn_fwd: kv_steps needs the partial-tile bitmaps");
    PA_CHECK_ARG(x->steps_pitch >= 1 && x->steps_pitch >= (x->pitch * x->A + 63) / 64,
                 "pa_attn_fwd: steps_pitch=%lld < max(1, %lld) (every list's first descriptor is read)",
                 (long long)x->steps_pitch, (long long)((x->pitch * x->A + 63) / 64));
    PA_CHECK_ARG((reinterpret_cast<uintptr_t>(x->kv_steps) & 15) == 0, "pa_attn_fwd: kv_steps not 16-byte aligned");
    {
      // row offsets inside a head are 32-bit in the streaming kernel
      const int64_t rb = (x->k_sn > x->v_sn ? x->k_sn : x->v_sn) * 2;
      PA_CHECK_ARG(x->N * rb < (1ll << 31), "pa_attn_fwd: N * row stride too large for kv_steps");
      PA_CHECK_ARG(!x->prev_o || x->prev_dtype == PA_F32 || x->N * x->prev_sn * 2 < (1ll << 31),
                   "pa_attn_fwd: N * prev row stride too large for kv_steps");
    }
    return pa::launch_attn_stream(a, x->dtype, s);
  }
  switch (x->dtype) {
    case PA_BF16: return pa::launch_attn_bf16(a, x->D, NW, s);
    case PA_F16: return pa::launch_attn_f16(a, x->D, NW, s);
    default: return pa::launch_attn_f32(a, x->D, NW, s);
  }
}

extern "C" int pa_attn_fwd_split(const pa_split_args* x, void* stream) {
  PA_CHECK_ARG(x && x->first && x->second, "pa_attn_fwd_split: null arguments");
  const pa_attn_args* f = x->first;
  const pa_attn_args* g = x->second;
  pa::AttnK a, b;
  if (int rc = pa::fill_attn(f, a)) return rc;
  if (int rc = pa::fill_attn(g, b)) return rc;
  const bool grid = x->items != nullptr;
  if (grid) {
    // one work-group per item: each piece's own descriptors (index order) and bitmaps
    PA_CHECK_ARG(x->n_items >= 1 && x->n_items <= 0x7fffffff, "pa_attn_fwd_split: n_items=%lld",
                 (long long)x->n_items);
    for (const pa_attn_args* y : {f, g}) {
      PA_CHECK_ARG(y->run_groups == 0 && y->kv_steps && !y->qblock_order,
                   "pa_attn_fwd_split: a grid split takes each piece's kv_steps in index order (no run, no order)");
      PA_CHECK_ARG(y->dtype == PA_BF16 || y->dtype == PA_F16, "pa_attn_fwd_split: f16 or bf16 only");
      PA_CHECK_ARG(y->D == 128 && y->BQ == 128 && (y->A == 16 || y->A == 32 || y->A == 64),
                   "pa_attn_fwd_split: D = 128, BQ = 128, A in 16, 32, 64");
      PA_CHECK_ARG(y->pitch == 0 || y->kv_bits, "pa_attn_fwd_split: the partial-tile bitmaps are needed");
      PA_CHECK_ARG(!(y->gather_q || y->scatter_o || y->gather_kv) || y->residue_s > 0,
                   "pa_attn_fwd_split: gathers and scatters go through the closed-form residue basis");
      PA_CHECK_ARG(y->steps_pitch >= 1 && y->steps_pitch >= (y->pitch * y->A + 63) / 64,
                   "pa_attn_fwd_split: steps_pitch too small");
      PA_CHECK_ARG((reinterpret_cast<uintptr_t>(y->kv_steps) & 15) == 0, "pa_attn_fwd_split: kv_steps alignment");
      const int64_t rb = (y->k_sn > y->v_sn ? y->k_sn : y->v_sn) * 2;
      PA_CHECK_ARG(y->N * rb < (1ll << 31) && y->N * y->o_sn * 2 < (1ll << 31),
                   "pa_attn_fwd_split: N * row stride too large");
    }
  } else {
    PA_CHECK_ARG(f->run_groups > 0 && g->run_groups == f->run_groups && x->run_groups == f->run_groups &&
                     f->run_steps == x->run_steps && g->run_steps == x->run_steps && f->run_start == x->run_start &&
                     g->run_start == x->run_start,
                 "pa_attn_fwd_split: both pieces must be run launches over the split's run rows");
  }
  PA_CHECK_ARG(f->q == g->q && f->k == g->k && f->v == g->v && f->o == g->o && f->lse == g->lse &&
                   f->q_sb == g->q_sb && f->q_sn == g->q_sn && f->k_sb == g->k_sb && f->k_sn == g->k_sn &&
                   f->v_sb == g->v_sb && f->v_sn == g->v_sn && f->o_sb == g->o_sb && f->o_sn == g->o_sn &&
                   f->lse_sb == g->lse_sb && f->BH == g->BH && f->N == g->N && f->D == g->D &&
                   f->dtype == g->dtype && f->scale == g->scale && f->BQ == g->BQ && f->A == g->A,
               "pa_attn_fwd_split: the pieces differ in tensors, shapes, dtype, scale or tile");
  PA_CHECK_ARG(f->lse && !f->prev_o, "pa_attn_fwd_split: the first piece writes o and lse (no prev_o)");
  PA_CHECK_ARG(g->prev_o == f->o && g->prev_lse == f->lse && g->prev_dtype == f->dtype && g->prev_sb == f->o_sb &&
                   g->prev_sn == f->o_sn,
               "pa_attn_fwd_split: the second piece merges into the first piece's o and lse");
  PA_CHECK_ARG(grid || x->kv_bits || (f->pitch == 0 && g->pitch == 0), "pa_attn_fwd_split: null kv_bits");
  PA_CHECK_ARG(x->sync && x->status && x->sync_groups >= 1 && x->sync_signal >= 1 && x->sync_wait >= 1,
               "pa_attn_fwd_split: sync=%p status=%p groups=%d signal=%d wait=%d", (void*)x->sync,
               (void*)x->status, x->sync_groups, x->sync_signal, x->sync_wait);
  if (!grid) a.kv_bits = x->kv_bits;
  a.run_res[1] = b.run_res[0];
  a.run_qlog2[1] = b.run_qlog2[0];
  a.run_flags[1] = b.run_flags[0];
  a.prev_o = b.prev_o;
  a.prev_dtype = b.prev_dtype;
  a.prev_sb = b.prev_sb;
  a.prev_sn = b.prev_sn;
  a.prev_lse = b.prev_lse;
  a.run_sync = x->sync;
  a.run_sync_groups = x->sync_groups;
  a.run_sync_signal = x->sync_signal;
  a.run_sync_wait = x->sync_wait;
  a.run_status = x->status;
  if (grid) {
    a.split_items = x->items;
    a.total_wg = x->n_items;
    a.steps1 = g->kv_steps;
    a.steps_pitch1 = g->steps_pitch;
    a.kv_bits1 = g->kv_bits;
    return pa::launch_attn_split_grid(a, f->dtype, static_cast<hipStream_t>(stream));
  }
  return pa::launch_attn_run(a, x->run_groups, f->dtype, true, static_cast<hipStream_t>(stream));
}
