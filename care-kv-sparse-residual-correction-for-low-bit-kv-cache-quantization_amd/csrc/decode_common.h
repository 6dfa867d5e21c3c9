// Shared definitions of the decode kernels: streaming pass, select, apply,
// combine (launched in that order on one stream; each kernel boundary
// orders the workspace writes of the previous kernel).
#pragma once

#include "common.h"

namespace carekv {

// Pages per split of the prefill correction's streaming pass over blocks of
// rows (pf_rows_stream_kernel): every work-group's serial chain of tiles
// stays this short, however long the prompt.
constexpr int kPfSplit = 32;

struct DecodeArgs {
  const uint16_t* q;
  uint16_t* out;
  const int32_t* seq_slot;
  const int32_t* n_pages;
  float* pml;          // [B*Hkv][nsplit][16][2]  split max (base-2 logits) / sum
  float* po;           // [B*Hkv][nsplit][16][D]  split unnormalised O
  float* rec;          // [B*Hkv][GQ][Pmax][F]    per-page records
  uint16_t* ebuf;      // [B*Hkv][GQ][Pmax][16]   fp16 e = 2^(x - m_ref) per token (correction on)
  float* scores;       // [B*Hkv][GQ][ncand]      candidate scores
  uint8_t* mask;       // [B*Hkv][GQ][Pmax]       selected slots per page
  float* ml;           // [B*Hkv][GQ][2]          global max (base 2) / sum
  float* num;          // [B*Hkv][nsplit][GQ][D]  apply partial numerators
  float* den;          // [B*Hkv][nsplit][GQ]     apply partial denominators
  float* xbuf;         // [B*Hkv][GQ][Pmax][16]   fp32 base-2 logits x (sketch proxy, adaptive policy)
  float* prox;         // [B*Hkv][GQ][Pmax][4]    mass, boundary, vdiff (sketch proxy only)
  float* xmax;         // [B*Hkv][nsplit][4][16]  prefill rows with the sketch proxy: each wave's
                       //                         maximum base-2 logit per query column
  const float* sketch_proj;  // [32][sketch_dim] fp32 (sketch proxy only)
  int32_t* diag;
  int32_t* err_flag;
  unsigned long long* read_counts;  // optional [3]: K reads, V reads, corrected queries
  int diag_cap;
  int B, Hq, GQ, nsplit, SP, Pmax, k_cap, v_cap, F, ncand;
  float sm_scale, sm_log2, sens, k_corr_scale, lam_k, lam_v, inv_sqrt_d;
  int correction, kind, joint, normalize, k_exact, budget_ratio, abs_k, abs_v;
  int SPA, napply;  // apply pass: pages per chunk (a multiple of SP) and chunk count (<= nsplit)
  // One launch of the streaming / proxy / apply kernels covers range 0: all
  // pages of each row, or on a packed KIVI arena range 1: the packed prefix
  // (pages below the row's n_packed) or range 2: the fp16 tail (the pages
  // from n_packed on).  Its grid has nsplit_run splits (napply_run chunks),
  // whose split partials go to slots split_base.. (chunk partials to
  // chunk_base..) of the nsplit (napply) the select and combine kernels read.
  int range, split_base, nsplit_run, chunk_base, napply_run;
  int proxy;        // 1: K scores from the sketch proxy (prox records), 0: from the moments
  int policy;       // 0 separate, 1 joint, 2 k_first, 3 adaptive (ResidualRouter.route)
  int adaptive_score, min_keep;  // read_budget_mode adaptive_score and its floor
  double ratio_k, ratio_v, sens_d, rel_thr, abs_thr;
  // byte span of the workspace from rec to the end of xbuf (< 4 GiB), and
  // the offsets of ebuf and xbuf from rec: one buffer resource covers them
  uint32_t ws_span, ws_e_off, ws_x_off;
  // Prefill rows (carekv_prefill_correct): batch entry b is row pf_row0 + b
  // of the prompt held by sequence pf_seq; it sees the prompt's first
  // pf_row0 + b + 1 tokens.  The streaming and apply passes read the
  // prompt's dense fp16 K_hat / V_hat (pf_k / pf_v, [Hkv][pf_T][D])
  // instead of the cache codes; the weights are half(2^(x - lse2)) with the
  // row's base-2 log-sum-exp (pf_lse, natural log, [Hq][pf_T]) as the
  // reference's fp16 attention weights; every candidate of the prompt's
  // pf_pages pages counts towards the normalisation and the budgets.
  // Entry b packs pf_R consecutive rows: its GQ = pf_G0 * pf_R query
  // columns are (row pf_row0 + b * pf_R + c / pf_G0, head c % pf_G0 of the
  // kv head's group); rows from pf_row_end on are padding.
  int pf;
  // prefill rows through pf_rows_stream_kernel (blocks of 4 entries, splits
  // of SP pages) rather than the entry-by-entry streaming kernel
  int pf_rows;
  int pf_seq, pf_row0, pf_row_end, pf_R, pf_G0, pf_pages, pf_T;
  const uint16_t* pf_k;
  const uint16_t* pf_v;
  const float* pf_lse;
  float* pf_vsq;  // [Hkv][pf_pages] sum of V_hat^2 over each page's prompt rows
  // [Hkv][3][pf_pages + 1]: over pages p .. pf_pages-1, the K slots and V
  // blocks a row seeing pages 0 .. p-1 counts without scoring (each page
  // capped at k_cap / v_cap as the select kernels count it), and 1 when one
  // of those pages holds more than the caps
  const int* pf_suf;
};

// The cache row and visible extent of batch entry b (for prefill rows, of
// its last row).
struct EntryRow {
  int seq, np, ntok;
};
__device__ __forceinline__ EntryRow entry_row(const carekv_arena& A, const DecodeArgs& a, int b) {
  EntryRow e;
  if (a.pf) {
    const int row = min(a.pf_row0 + (b + 1) * a.pf_R, a.pf_row_end) - 1;
    e.seq = a.pf_seq;
    e.ntok = row + 1;
    e.np = row / kPage + 1;
  } else {
    const int s = a.seq_slot[b], n = a.n_pages[b];
    const bool ok = s >= 0 && s < A.n_seq && n >= 0 && n <= a.Pmax;
    e.seq = ok ? s : 0;
    e.np = ok ? n : 0;
    e.ntok = 0x7fffffff;
  }
  return e;
}

// Pages [lo, hi) of a row of np pages that a launch covers (DecodeArgs::range).
__device__ __forceinline__ void launch_pages(const carekv_arena& A, const DecodeArgs& a, int seq, int np, int& lo,
                                             int& hi) {
  lo = 0;
  hi = np;
  if (a.range != 0) {
    const int off = min(max(A.n_packed[seq], 0), np);
    if (a.range == 1) hi = off;
    else lo = off;
  }
}

// Query column c of prefill entry b of kv head kvh: its prompt row, its
// query head, and whether the row exists.
struct PfCol {
  int row, head;
  bool ok;
};
__device__ __forceinline__ PfCol pf_col(const DecodeArgs& a, int b, int kvh, int c) {
  PfCol x;
  x.row = a.pf_row0 + b * a.pf_R + c / a.pf_G0;
  x.head = kvh * a.pf_G0 + c % a.pf_G0;
  x.ok = c < a.GQ && x.row < a.pf_row_end;
  return x;
}
// Split partials of entry b that hold data: all of them, except in the
// prefill rows pass, which writes no partial for a split past the entry's
// last page (its rows see pages 0 .. row / kPage).
__device__ __forceinline__ int splits_read(const DecodeArgs& a, int b) {
  if (!a.pf_rows) return a.nsplit;
  const int row = min(a.pf_row0 + (b + 1) * a.pf_R, a.pf_row_end) - 1;
  return min(a.nsplit, (row / kPage + a.SP) / a.SP);
}
// Element offset of a column's row in q / out / diag rows ([n_rows][Hq][.]).
__device__ __forceinline__ long pf_row_off(const DecodeArgs& a, const PfCol& x) {
  return (long)(x.row - a.pf_row0) * a.Hq + x.head;
}

// Page record per (sequence, kv head, query, page), F = 2 + 4*k_cap +
// v_cap floats:
//   [0]                      m_ref: running max of the base-2 logits
//                            x = s * log2(e) at the page
//   [1 + 4r .. 3 + 4r]       M2, M3, M4 of the r-th stored K slot (cg order)
//   [4 + 4r]                 D*: dS_t*^2 of the r-th stored K slot
//   [1 + 4*k_cap]            e_t*
//   [2 + 4*k_cap + r]        sum_t e_t over the r-th stored V block
// with e_t = 2^(x_t - m_ref), t* the page's first token of largest e_t, and
// Mk = sum_t dS_t^2 e_t^k over the page's valid tokens other than t*.  The
// K score sum_t dS_t^2 a_t^2 (1 - a_t)^2 (a_t = c e_t) is then
// c^2 [M2 - 2 c M3 + c^2 M4 + D* (e* (1 - c e*))^2]: the one token whose a_t
// can exceed 1/2 (where the expansion cancels) is evaluated directly, as
// the reference evaluates A (1 - A), and the select kernel keeps c outside
// the square root (c^2 of a page far below the maximum underflows fp32
// where the reference's per-token terms do not).  Written only for pages
// with metadata.
//
// ebuf holds the page's e_t (0 past the valid tokens) for the apply pass.
// With the sketch proxy the K moments are not written; xbuf holds the
// page's x_t (-inf past the valid tokens) and decode_proxy_kernel turns
// them into the prox records.
//
// Selection mask per (sequence, kv head, query, page): bit r = the r-th
// stored K slot of the page is selected, bit 4 + r = the r-th stored V block.

int launch_decode_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);
int launch_decode_stream4(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);  // GQ <= 4, SP % 16 == 0
int launch_pf_rows_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);  // prefill rows, one split
int launch_decode_proxy(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);
int launch_decode_select(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);
int launch_decode_apply(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);
int launch_decode_apply4(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);  // GQ <= 4
int launch_decode_combine(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);

}  // namespace carekv
