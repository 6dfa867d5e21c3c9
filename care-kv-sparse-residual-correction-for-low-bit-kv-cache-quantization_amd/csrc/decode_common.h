// Shared definitions of the two decode kernels (streaming pass, finalize).
#pragma once

#include "common.h"

namespace carekv {

struct DecodeArgs {
  const uint16_t* q;
  uint16_t* out;
  const int32_t* seq_slot;
  const int32_t* n_pages;
  float* pml;          // [B*Hkv][nsplit][16][2]  split max / sum
  float* po;           // [B*Hkv][nsplit][16][D]  split unnormalised O
  float* rec;          // [B*Hkv][Pmax][GQ][F]    per-page records
  float* scores;       // [B*Hkv][GQ][ncand]
  int32_t* sel;        // [B*Hkv][GQ][ncand]
  int32_t* diag;
  int32_t* err_flag;
  int diag_cap;
  int B, Hq, GQ, nsplit, SP, Pmax, k_cap, v_cap, F, ncand;
  float sm_scale, sens, k_corr_scale, lam_k, lam_v, sqrt_d;
  int correction, kind, joint, normalize, k_exact, budget_ratio, abs_k, abs_v;
  double ratio_k, ratio_v, sens_d;
};

// Page record layout per (sequence, kv head, page, query):
//   [0]                      m_ref: logit reference (running max) of the page
//   [1 + 3r .. 3 + 3r]       M2, M3, M4 of the r-th stored K slot (cg order)
//   [1 + 3*k_cap + r]        sum_t exp(s_t - m_ref) over the r-th stored V block
// with Mk = sum_t dS_t^2 exp(s_t - m_ref)^k over the page's valid tokens.

int launch_decode_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);
int launch_decode_finalize(const carekv_arena& A, const DecodeArgs& a, hipStream_t s);

}  // namespace carekv
