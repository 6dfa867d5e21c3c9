// C ABI of the decode path: workspace layout, argument checks, launches of
// the streaming, select, apply and combine kernels on the caller's stream.
#include <mutex>

#include "block_util.h"
#include "decode_common.h"
#include "host_util.h"

using namespace carekv;

namespace {
struct WsLayout {
  long err, pml, po, rec, ebuf, scores, mask, ml, num, den, xbuf, prox, xmax, total;
  int nsplit, F, ncand;
};

// gq: query columns per (entry, kv head); 0 = n_heads / n_kv_heads; pf:
// prefill rows
WsLayout ws_layout(const carekv_arena& A, const carekv_decode_params& dp, int gq = 0, bool pf = false) {
  WsLayout L{};
  const long BH = (long)dp.batch * A.n_kv_heads;
  const int GQ = gq > 0 ? gq : dp.n_heads / A.n_kv_heads;
  const int D = A.head_dim;
  const int Pm = dp.max_pages_used > 0 ? dp.max_pages_used : 1;
  L.nsplit = (Pm + dp.split_pages - 1) / dp.split_pages;
  if (A.kivi_packed && !pf) {  // the packed prefix and the fp16 tail split apart
    const int pp = dp.packed_pages_used > 0 ? dp.packed_pages_used : 0;
    const int tp = dp.tail_pages_used > 0 ? dp.tail_pages_used : 0;
    L.nsplit = (pp + dp.split_pages - 1) / dp.split_pages + (tp + dp.split_pages - 1) / dp.split_pages;
    if (L.nsplit == 0) L.nsplit = 1;
  }
  L.F = 2 + 4 * dp.k_cap + dp.v_cap;
  L.ncand = Pm * (dp.k_cap + dp.v_cap);
  auto al = [](long x) { return (x + 255) / 256 * 256; };
  long off = 0;
  L.err = off; off += 256;
  L.pml = off; off += al(BH * L.nsplit * 16 * 2 * 4);
  L.po = off; off += al(BH * L.nsplit * 16 * (long)D * 4);
  L.rec = off; off += al(BH * GQ * (long)Pm * L.F * 4);
  L.ebuf = off; off += al(BH * GQ * (long)Pm * 16 * 2);
  L.scores = off; off += al(BH * GQ * (long)L.ncand * 4);
  L.mask = off; off += al(BH * GQ * (long)Pm);
  L.ml = off; off += al(BH * GQ * 2 * 4);
  L.num = off; off += al(BH * L.nsplit * GQ * (long)D * 4);
  L.den = off; off += al(BH * L.nsplit * GQ * 4);
  const bool proxy = dp.k_proxy != 0 && dp.correction != 0;
  const bool need_x = dp.correction != 0 && (dp.k_proxy != 0 || dp.route_policy == 3);
  L.xbuf = off; off += need_x ? al(BH * GQ * (long)Pm * 16 * 4) : 0;
  L.prox = off; off += proxy ? al(BH * GQ * (long)Pm * 4 * 4) : 0;
  L.xmax = off; off += (pf && proxy) ? al(BH * L.nsplit * 4 * 16 * 4) : 0;
  L.total = off;
  return L;
}
}  // namespace

extern "C" int64_t carekv_decode_workspace_bytes(const carekv_arena* arena, const carekv_decode_params* dp) {
  if (!arena || !dp || dp->split_pages <= 0 || arena->n_kv_heads <= 0) return -1;
  return ws_layout(*arena, *dp).total;
}

namespace {
// Prefill rows of carekv_prefill_correct (null for a decode step).
struct PfRows {
  const carekv_prefill_corr_params* p;
  int pages;
  int R, G0;  // rows per entry, query heads per kv head
  bool rows;  // the streaming pass over blocks of entries (pf_rows_stream_kernel)
};

__global__ __launch_bounds__(256) void prompt_vsq_kernel(const uint16_t* __restrict__ v, int T, int D, int pages,
                                                         float* __restrict__ vsq) {
  // one wave per (page, kv head): sum of V_hat^2 over the page's prompt rows
  const int p = blockIdx.x * 4 + (threadIdx.x >> 6), kvh = blockIdx.y;
  const int lane = threadIdx.x & 63;
  if (p >= pages) return;
  const int r1 = min(T, (p + 1) * kPage);
  float acc = 0.f;
  for (int r = p * kPage; r < r1; ++r)
    for (int d = lane; d < D; d += 64) {
      const float x = h2f(v[((long)kvh * T + r) * D + d]);
      acc = fmaf(x, x, acc);
    }
  acc = wave_sum_f(acc);
  if (lane == 0) vsq[(long)kvh * pages + p] = acc;
}

// The candidates of the prompt's later pages, per kv head, as suffix counts
// over the pages (DecodeArgs::pf_suf): the select kernels read them at a
// row's page count instead of walking the pages past the row.  Page p
// counts when it holds valid rows and metadata: min(stored K slots, k_cap),
// its stored V blocks of rank < v_cap that start inside the valid rows, and
// an overflow when it holds more K slots than k_cap or more V blocks than
// v_cap.  One work-group per kv head, chunks of 256 pages from the end.
__global__ __launch_bounds__(256) void prompt_suffix_kernel(carekv_arena A, int seq, int pages, int k_cap, int v_cap,
                                                            int* __restrict__ suf) {
  __shared__ BlockScratch bs;
  const int kvh = blockIdx.x, tid = threadIdx.x;
  const int ncg = A.head_dim / 32;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  int* sk = suf + (long)kvh * 3 * (pages + 1);
  int* sv = sk + (pages + 1);
  int* so = sv + (pages + 1);
  if (tid == 0) { sk[pages] = 0; sv[pages] = 0; so[pages] = 0; }
  int ck = 0, cv = 0, co = 0;  // totals of the pages from hi on
  for (int hi = pages; hi > 0; hi -= kBlock) {
    const int p = hi - 1 - tid;  // descending with the thread index
    int nk = 0, nvb = 0, ov = 0;
    if (p >= 0) {
      const long pg = pg_base + p;
      const int nv = A.valid[pg];
      if (nv > 0 && A.has_meta[pg]) {
        int rk = 0;
        for (int cg = 0; cg < ncg; ++cg) {
          const int sl = A.k_slot[pg * ncg + cg];
          rk += (sl >= 0 && sl < A.n_slots) ? 1 : 0;
        }
        ov = rk > k_cap ? 1 : 0;
        nk = min(rk, k_cap);
        int rv = 0;
        for (int vb = 0; vb < kVtb; ++vb) {
          const int sl = A.v_slot[pg * kVtb + vb];
          if (!(sl >= 0 && sl < A.n_slots)) continue;
          if (rv >= v_cap) { ov = 1; break; }
          if (vb * kVtb < nv) ++nvb;
          ++rv;
        }
      }
    }
    // exclusive scans over the thread index = the chunk's pages above p
    int tk, tv, to;
    const int ek = block_excl_scan(nk, bs, &tk);
    const int ev = block_excl_scan(nvb, bs, &tv);
    const int eo = block_excl_scan(ov, bs, &to);
    if (p >= 0) {
      sk[p] = ck + ek + nk;
      sv[p] = cv + ev + nvb;
      so[p] = (co + eo + ov) > 0 ? 1 : 0;
    }
    ck += tk; cv += tv; co += to;
  }
}

// Workspace bytes a prefill-rows call needs beyond the decode layout: v_sq
// per (kv head, page), then the suffix counts.
long pf_extra_bytes(const carekv_arena& A, int pages) {
  const long vsq = ((long)A.n_kv_heads * pages * 4 + 255) / 256 * 256;
  return vsq + (long)A.n_kv_heads * 3 * (pages + 1) * 4;
}

int run_decode(const carekv_arena* arena, const carekv_decode_params* dp, const PfRows* pf, const uint16_t* q,
               uint16_t* out, void* workspace, int64_t workspace_bytes, int32_t* diag, int32_t diag_cap,
               void* stream) {
  CAREKV_REQUIRE(arena && dp && q && out && workspace, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.residual_bits == 4, "kernels support residual_bits=4");
  CAREKV_REQUIRE(dp->batch > 0 && dp->n_heads > 0, "batch and n_heads must be positive");
  CAREKV_REQUIRE(dp->n_heads % A.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
  const int GQ = pf ? pf->G0 * pf->R : dp->n_heads / A.n_kv_heads;
  CAREKV_REQUIRE(GQ >= 1 && GQ <= 16, "query heads per kv head must be in 1..16");
  CAREKV_REQUIRE(pf || (dp->seq_slot && dp->n_pages), "seq_slot and n_pages are required");
  CAREKV_REQUIRE(dp->max_pages_used >= 0 && dp->max_pages_used <= A.max_pages, "max_pages_used out of range");
  CAREKV_REQUIRE(dp->split_pages > 0 && dp->split_pages % 4 == 0 && dp->split_pages <= 1024,
                 "split_pages must be a multiple of 4 in 4..1024");
  CAREKV_REQUIRE(dp->k_cap >= 0 && dp->k_cap <= A.head_dim / 32, "k_cap out of range");
  CAREKV_REQUIRE(dp->v_cap >= 0 && dp->v_cap <= 4, "v_cap out of range");
  CAREKV_REQUIRE(dp->lambda_k > 0.f && dp->lambda_v > 0.f, "KSCORE lambdas must be positive");
  CAREKV_REQUIRE(!diag || diag_cap > 0, "diag_cap must be positive");
  const bool proxy = dp->k_proxy != 0 && dp->correction != 0;
  CAREKV_REQUIRE(!proxy || dp->sketch_proj, "the sketch proxy needs sketch_proj");
  CAREKV_REQUIRE(dp->route_policy == 0 || dp->route_policy == 2 || dp->route_policy == 3,
                 "route_policy must be 0 (joint flag), 2 (k_first) or 3 (adaptive)");
  CAREKV_REQUIRE(dp->min_keep >= 0, "min_keep must be non-negative");
  const bool need_x = dp->correction != 0 && (proxy || dp->route_policy == 3);
  CAREKV_REQUIRE(!proxy || (A.k_sketch && A.k_channel_group == 32 && A.sketch_dim >= 1 && A.sketch_dim <= 64),
                 "the sketch proxy needs k_sketch, k_channel_group 32 and sketch_dim in 1..64");
  const bool kv = A.kivi_packed != 0 && !pf;
  if (kv) {
    CAREKV_REQUIRE(GQ <= 4 && dp->split_pages % 16 == 0,
                   "a packed KIVI arena decodes with at most 4 query heads per kv head and split_pages a "
                   "multiple of 16");
    CAREKV_REQUIRE(dp->packed_pages_used >= 0 && dp->tail_pages_used >= 0 &&
                       dp->packed_pages_used <= A.max_pages && dp->tail_pages_used <= A.tail_pages,
                   "packed_pages_used / tail_pages_used out of range");
  }
  const WsLayout L = ws_layout(A, *dp, GQ, pf != nullptr);
  const long vsq_off = L.total, need = L.total + (pf ? pf_extra_bytes(A, pf->pages) : 0);
  if (workspace_bytes < need) {
    set_error("%s: workspace too small (%lld < %lld)", pf ? "carekv_prefill_correct" : "carekv_decode_attn",
              (long long)workspace_bytes, (long long)need);
    return CAREKV_ESPACE;
  }
  CAREKV_REQUIRE(L.prox - L.rec < (1L << 32) - 256,
                 "workspace from the records to the logits exceeds 4 GiB: lower batch or max_pages_used");
  char* ws = (char*)workspace;
  DecodeArgs a{};
  a.q = q; a.out = out; a.seq_slot = dp->seq_slot; a.n_pages = dp->n_pages;
  a.err_flag = (int32_t*)(ws + L.err);
  a.pml = (float*)(ws + L.pml);
  a.po = (float*)(ws + L.po);
  a.rec = (float*)(ws + L.rec);
  a.ebuf = (uint16_t*)(ws + L.ebuf);
  a.scores = (float*)(ws + L.scores);
  a.mask = (uint8_t*)(ws + L.mask);
  a.ml = (float*)(ws + L.ml);
  a.num = (float*)(ws + L.num);
  a.den = (float*)(ws + L.den);
  a.proxy = proxy ? 1 : 0;
  a.xbuf = need_x ? (float*)(ws + L.xbuf) : nullptr;
  a.policy = dp->route_policy == 0 ? (dp->joint ? 1 : 0) : dp->route_policy;
  a.adaptive_score = dp->adaptive_score != 0;
  a.rel_thr = dp->rel_threshold; a.abs_thr = dp->abs_threshold; a.min_keep = dp->min_keep;
  a.prox = proxy ? (float*)(ws + L.prox) : nullptr;
  a.xmax = (pf && proxy) ? (float*)(ws + L.xmax) : nullptr;
  a.ws_span = (uint32_t)(L.prox - L.rec);
  a.ws_e_off = (uint32_t)(L.ebuf - L.rec);
  a.ws_x_off = (uint32_t)(L.xbuf - L.rec);
  a.sketch_proj = dp->sketch_proj;
  a.diag = diag; a.diag_cap = diag_cap;
  a.read_counts = dp->read_counts;
  a.B = dp->batch; a.Hq = dp->n_heads; a.GQ = GQ; a.nsplit = L.nsplit; a.SP = dp->split_pages;
  a.Pmax = dp->max_pages_used > 0 ? dp->max_pages_used : 1;
  a.k_cap = dp->k_cap; a.v_cap = dp->v_cap; a.F = L.F; a.ncand = L.ncand;
  a.sm_scale = dp->sm_scale; a.sens = dp->sensitivity; a.sens_d = (double)dp->sensitivity;
  a.k_corr_scale = dp->k_corr_scale;
  // the KSCORE lambdas weigh the normalised scores of the live selector of
  // vectorized_joint_correction only (attention.py:838-844); the router's
  // policies and thresholds have none
  const bool no_lam = proxy || dp->route_policy >= 2 || dp->adaptive_score;
  a.lam_k = no_lam ? 1.f : dp->lambda_k; a.lam_v = no_lam ? 1.f : dp->lambda_v;
  a.sm_log2 = (float)((double)dp->sm_scale * 1.4426950408889634074);  // log2(e)
  a.inv_sqrt_d = (float)(1.0 / sqrt((double)A.head_dim));
  a.correction = dp->correction; a.kind = dp->kind; a.joint = dp->joint; a.normalize = dp->normalize;
  a.k_exact = dp->k_exact; a.budget_ratio = dp->budget_ratio; a.abs_k = dp->abs_k; a.abs_v = dp->abs_v;
  a.ratio_k = dp->ratio_k; a.ratio_v = dp->ratio_v;
  // splits and apply chunks of the packed prefix (range 1) and the fp16
  // tail (range 2) of a packed KIVI arena; one range (0) otherwise
  int ns_p = L.nsplit, ns_t = 0, na_p = 0, na_t = 0;
  if (kv) {
    ns_p = (dp->packed_pages_used + a.SP - 1) / a.SP;
    ns_t = L.nsplit - ns_p;
  }
  {  // apply chunks: the largest power-of-two multiple of the split (at most
     // 1024 pages) that still gives >= 1024 work-groups, which every CU holds
     // at once; fewer, longer chunks amortise the per-work-group item scan
    const long pairs = (long)a.B * A.n_kv_heads;
    int m = 1;
    while (a.SP * 2 * m <= 1024 && pairs * ((a.nsplit + 2 * m - 1) / (2 * m)) >= 1024) m *= 2;
    a.SPA = a.SP * m;
    na_p = (ns_p + m - 1) / m;
    na_t = (ns_t + m - 1) / m;
    a.napply = na_p + na_t;
  }
  // the tail view: the fp16 side-buffer rows of tail_k / tail_v under the
  // code-page map of n_packed
  carekv_arena At = A;
  if (kv) {
    At.base_bits = 16;
    At.scale_mode = 0;
    At.kcodes = (int8_t*)A.tail_k;
    At.vcodes = (int8_t*)A.tail_v;
    At.kivi_packed = 0;
    At.code_pages = A.tail_pages;
    At.code_page_off = A.n_packed;
  }
  // one call per range with pages (the prefix first: its first split clears the status word)
  auto ranges = [&](auto&& launch, bool chunks) -> int {
    if (!kv) {
      a.range = 0; a.split_base = 0; a.nsplit_run = a.nsplit; a.chunk_base = 0; a.napply_run = a.napply;
      return launch(A);
    }
    int rc = CAREKV_OK;
    const int n_p = chunks ? na_p : ns_p, n_t = chunks ? na_t : ns_t;
    if (n_p > 0) {
      a.range = 1; a.split_base = 0; a.nsplit_run = ns_p; a.chunk_base = 0; a.napply_run = na_p;
      rc = launch(A);
    }
    if (rc == CAREKV_OK && n_t > 0) {
      a.range = 2; a.split_base = ns_p; a.nsplit_run = ns_t; a.chunk_base = na_p; a.napply_run = na_t;
      rc = launch(At);
    }
    a.range = 0;
    return rc;
  };
  hipStream_t s = (hipStream_t)stream;
  if (pf) {
    const carekv_prefill_corr_params& P = *pf->p;
    a.pf = 1;
    a.pf_rows = pf->rows ? 1 : 0;
    a.pf_seq = P.seq; a.pf_row0 = P.row_begin; a.pf_row_end = P.row_begin + P.n_rows;
    a.pf_R = pf->R; a.pf_G0 = pf->G0; a.pf_pages = pf->pages; a.pf_T = P.n_tokens;
    a.pf_k = P.k_hat; a.pf_v = P.v_hat; a.pf_lse = P.lse;
    a.pf_vsq = (float*)(ws + vsq_off);
    hipLaunchKernelGGL(prompt_vsq_kernel, dim3((unsigned)((pf->pages + 3) / 4), A.n_kv_heads), dim3(256), 0, s,
                       P.v_hat, P.n_tokens, A.head_dim, pf->pages, a.pf_vsq);
    CAREKV_CHECK_LAUNCH("prompt_vsq");
    int* suf = (int*)(ws + vsq_off + ((long)A.n_kv_heads * pf->pages * 4 + 255) / 256 * 256);
    a.pf_suf = suf;
    hipLaunchKernelGGL(prompt_suffix_kernel, dim3(A.n_kv_heads), dim3(kBlock), 0, s, A, P.seq, pf->pages, a.k_cap,
                       a.v_cap, suf);
    CAREKV_CHECK_LAUNCH("prompt_suffix");
  }
  hipEvent_t* ev = (hipEvent_t*)dp->phase_events;
  auto mark = [&](int i) -> int {
    if (ev && hipEventRecord(ev[i], s) != hipSuccess) {
      set_error("carekv_decode_attn: hipEventRecord failed on phase event %d", i);
      return CAREKV_ELAUNCH;
    }
    return CAREKV_OK;
  };
  int rc = mark(0);
  if (rc == CAREKV_OK) rc = ranges([&](const carekv_arena& V) { return launch_decode_stream(V, a, s); }, false);
  if (rc == CAREKV_OK) rc = mark(1);
  if (rc == CAREKV_OK && proxy)
    rc = ranges([&](const carekv_arena& V) { return launch_decode_proxy(V, a, s); }, false);
  if (rc == CAREKV_OK) rc = launch_decode_select(A, a, s);
  if (rc == CAREKV_OK) rc = mark(2);
  if (rc == CAREKV_OK && a.correction)
    rc = ranges([&](const carekv_arena& V) { return launch_decode_apply(V, a, s); }, true);
  if (rc == CAREKV_OK) rc = mark(3);
  if (rc == CAREKV_OK && a.correction) rc = launch_decode_combine(A, a, s);
  if (rc == CAREKV_OK) rc = mark(4);
  return rc;
}
}  // namespace

extern "C" int carekv_decode_attn(const carekv_arena* arena, const carekv_decode_params* dp, const uint16_t* q,
                                  uint16_t* out, void* workspace, int64_t workspace_bytes, int32_t* diag,
                                  int32_t diag_cap, void* stream) {
  return run_decode(arena, dp, nullptr, q, out, workspace, workspace_bytes, diag, diag_cap, stream);
}

namespace {
// The decode parameters of a prefill-rows call and its page count, or an
// error message.
int prefill_setup(const carekv_arena* arena, const carekv_decode_params* read,
                  const carekv_prefill_corr_params* pp, carekv_decode_params& dp, PfRows& pf) {
  CAREKV_REQUIRE(arena && read && pp, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(pp->seq >= 0 && pp->seq < A.n_seq, "seq out of range");
  CAREKV_REQUIRE(pp->n_tokens >= 1, "n_tokens must be positive");
  const int pages = (pp->n_tokens + kPage - 1) / kPage;
  CAREKV_REQUIRE(pages <= A.max_pages, "the prompt needs more pages than the arena holds");
  CAREKV_REQUIRE(pp->row_begin >= 0 && pp->n_rows >= 1 && pp->row_begin + pp->n_rows <= pp->n_tokens,
                 "rows must lie in [0, n_tokens)");
  CAREKV_REQUIRE(pp->k_hat && pp->v_hat && pp->lse, "k_hat, v_hat and lse are required");
  CAREKV_REQUIRE((long)pp->n_tokens * A.head_dim * 2 < (1L << 32), "prompt rows exceed 4 GiB per kv head");
  CAREKV_REQUIRE(read->correction != 0, "prefill rows run the correction (correction must be 1)");
  CAREKV_REQUIRE(read->n_heads > 0 && read->n_heads % A.n_kv_heads == 0 && read->n_heads / A.n_kv_heads <= 16,
                 "n_heads must be a multiple of n_kv_heads with at most 16 query heads per kv head");
  dp = *read;
  pf.p = pp;
  pf.pages = pages;
  // pack consecutive rows into the 16 query columns of an entry
  pf.G0 = read->n_heads / A.n_kv_heads;
  pf.R = 16 / pf.G0;
  dp.batch = (pp->n_rows + pf.R - 1) / pf.R;
  dp.max_pages_used = pages;
  // with the moments' K score the streaming pass runs on blocks of 4
  // entries (pf_rows_stream_kernel) in splits of kPfSplit pages, so that the
  // longest rows' serial chains stay short (at most 16 splits; the split's
  // pages are a multiple of 4).  CAREKV_PF_ROWS=0: entry by entry over the
  // caller's splits; CAREKV_PF_SPLIT overrides the pages per split.
  const char* env = getenv("CAREKV_PF_ROWS");
  pf.rows = !(env && env[0] == '0') && read->k_proxy == 0 && read->route_policy != 3 && pages <= 1024 &&
            (A.head_dim == 64 || A.head_dim == 128);
  if (pf.rows) {
    const char* es = getenv("CAREKV_PF_SPLIT");
    int sp = es ? atoi(es) : kPfSplit;
    sp = max(sp, (pages + 15) / 16);
    sp = min(max((sp + 3) / 4 * 4, 4), (pages + 3) / 4 * 4);
    dp.split_pages = sp;
  }
  dp.seq_slot = nullptr;
  dp.n_pages = nullptr;
  return CAREKV_OK;
}
}  // namespace

extern "C" int64_t carekv_prefill_correct_workspace_bytes(const carekv_arena* arena,
                                                          const carekv_decode_params* read,
                                                          const carekv_prefill_corr_params* pp) {
  carekv_decode_params dp{};
  PfRows pf{};
  if (prefill_setup(arena, read, pp, dp, pf) != CAREKV_OK || dp.split_pages <= 0) return -1;
  return ws_layout(*arena, dp, pf.G0 * pf.R, true).total + pf_extra_bytes(*arena, pf.pages);
}

extern "C" int carekv_prefill_correct(const carekv_arena* arena, const carekv_decode_params* read,
                                      const carekv_prefill_corr_params* pp, const uint16_t* q, uint16_t* out,
                                      void* workspace, int64_t workspace_bytes, int32_t* diag, int32_t diag_cap,
                                      void* stream) {
  carekv_decode_params dp{};
  PfRows pf{};
  const int rc = prefill_setup(arena, read, pp, dp, pf);
  if (rc != CAREKV_OK) return rc;
  return run_decode(arena, &dp, &pf, q, out, workspace, workspace_bytes, diag, diag_cap, stream);
}

// ------------------------------------------------------------------ no-allocation variant
// carekv_decode_attn_static: the decode step with its workspace in a
// file-scope device array instead of a caller buffer, for callers that
// cannot allocate (graph capture, tight serving loops).  Each GPU holds its
// own copy of the array for the life of the process; host code reaches it
// only through the address hipGetSymbolAddress returns on that device (the
// array's name is a host-side stand-in).  Calls that overlap on one GPU share
// the array and race.
namespace {
static __device__ __align__(256) char scratch[CAREKV_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per
// device), or null with the error message set.
void* static_scratch(int dev) {
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("carekv_decode_attn_static: device %d out of range", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("carekv_decode_attn_static: hipGetSymbolAddress failed on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}
}  // namespace

extern "C" int carekv_decode_attn_static(const carekv_arena* arena, const carekv_decode_params* dp,
                                         const uint16_t* q, uint16_t* out, int32_t* diag, int32_t diag_cap,
                                         void* stream) {
  CAREKV_REQUIRE(arena && dp, "null argument");
  CAREKV_REQUIRE(dp->split_pages > 0 && arena->n_kv_heads > 0, "split_pages and n_kv_heads must be positive");
  int dev = -1, sdev = -1;
  if (hipGetDevice(&dev) != hipSuccess || hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess) {
    set_error("carekv_decode_attn_static: cannot resolve the current device or the stream's device");
    return CAREKV_ELAUNCH;
  }
  CAREKV_REQUIRE(dev == sdev, "the stream's device must be the current device");
  const int64_t need = ws_layout(*arena, *dp).total;
  if (need > (int64_t)CAREKV_STATIC_SCRATCH_BYTES) {
    set_error("carekv_decode_attn_static: this step needs %lld workspace bytes, the static scratch holds %lld "
              "(CAREKV_STATIC_SCRATCH_BYTES): lower the batch or max_pages_used, or use carekv_decode_attn "
              "with a caller workspace", (long long)need, (long long)CAREKV_STATIC_SCRATCH_BYTES);
    return CAREKV_ESPACE;
  }
  void* ws = static_scratch(dev);
  if (!ws) return CAREKV_ELAUNCH;
  return run_decode(arena, dp, nullptr, q, out, ws, CAREKV_STATIC_SCRATCH_BYTES, diag, diag_cap, stream);
}
