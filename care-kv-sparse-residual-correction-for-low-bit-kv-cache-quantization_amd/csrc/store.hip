// Page writes (quantize + pack + int8 page scales), store-time residual
// candidates / selection / slot packing, and single-token decode appends.
//
// Reference semantics (paths relative to the reference root):
//   quantize (fp16 arithmetic)        quantizer.py:31-64
//   INT2/3/4 packing                  quantizer.py:257-372
//   int8 scale codes + fp16 master    cache.py:592-654, 689-695
//   process_page                      residual_store.py:239-464
//   4-bit residual slot packing       residual_store.py:121-136
//   decode append + store on fill     layer.py:1028-1146
#include "common.h"

namespace carekv {

struct StoreWs {  // per job: [0]=K count, [1]=V count, [2]=K base, [3]=V base
  int32_t* v;
};

// One wave quantizes one row group: 32 fp16 values -> codes, fp16 scale.
// fp16 chain of quantizer.py:51-59: max|x| (exact), scale=half(max/qmax),
// code=clamp(rint(half(x/scale))), NaN (0/0 on an all-zero group) -> 0.
template <int BITS>
__device__ __forceinline__ _Float16 quant_group(const float* x, int* code) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(x[i]));
  const _Float16 scale = (_Float16)(m / (float)qmax);
  const float sf = (float)scale;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float qh = (float)(_Float16)(x[i] / sf);
    float r = rintf(qh);
    r = fminf(fmaxf(r, (float)(-qmax - 1)), (float)qmax);
    code[i] = (qh != qh) ? 0 : (int)r;
  }
  return scale;
}

template <int BITS>
__device__ __forceinline__ void pack_group(const int* code, uint32_t* w) {
#pragma unroll
  for (int i = 0; i < BITS; ++i) w[i] = 0;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint32_t u = (uint32_t)code[k] & ((1u << BITS) - 1u);
    const int bit = BITS * k;
    w[bit >> 5] |= u << (bit & 31);
    if ((bit & 31) + BITS > 32) w[(bit >> 5) + 1] |= u >> (32 - (bit & 31));
  }
}

// int8 scale code of `s` against master `m` (cache.py:601-602, 692-693).
__device__ __forceinline__ int8_t scale_code(float s, float m) {
  const float q = s / m;
  if (q != q) return 0;
  return (int8_t)fminf(fmaxf(rintf(q), -128.f), 127.f);
}

// Store decision for one page: candidate order by prior (double, stable,
// descending), prior > 0 only, per-kind budgets or joint budget
// (residual_store.py:372-422).  sel_k/sel_v receive candidate indices in
// slot-allocation order; returns counts.
template <int NCG>
__device__ __forceinline__ void select_candidates(const float* kerr, const float* verr,
                                                  const carekv_store_params& sp, double struct_prior,
                                                  int* sel_k, int& nk, int* sel_v, int& nv, int* order_kind,
                                                  int* order_idx, int& n_order) {
  double pk[NCG], pv[kVtb];
  int ik[NCG], iv[kVtb];
#pragma unroll
  for (int i = 0; i < NCG; ++i) { pk[i] = (double)kerr[i] * sp.sensitivity * struct_prior; ik[i] = i; }
#pragma unroll
  for (int i = 0; i < kVtb; ++i) { pv[i] = (double)verr[i] * sp.sensitivity * struct_prior; iv[i] = i; }
  // stable insertion sort, descending
  for (int i = 1; i < NCG; ++i)
    for (int j = i; j > 0 && pk[j] > pk[j - 1]; --j) {
      double t = pk[j]; pk[j] = pk[j - 1]; pk[j - 1] = t;
      int u = ik[j]; ik[j] = ik[j - 1]; ik[j - 1] = u;
    }
  for (int i = 1; i < kVtb; ++i)
    for (int j = i; j > 0 && pv[j] > pv[j - 1]; --j) {
      double t = pv[j]; pv[j] = pv[j - 1]; pv[j - 1] = t;
      int u = iv[j]; iv[j] = iv[j - 1]; iv[j - 1] = u;
    }
  int pos_k = 0, pos_v = 0;
  for (int i = 0; i < NCG; ++i) pos_k += pk[i] > 0.0;
  for (int i = 0; i < kVtb; ++i) pos_v += pv[i] > 0.0;
  nk = nv = n_order = 0;
  if (sp.store_none) return;
  if (sp.joint) {
    // merge the two sorted positive lists, K before V on equal priors
    int a = 0, b = 0;
    while (n_order < sp.joint_budget && (a < pos_k || b < pos_v)) {
      const bool take_k = (b >= pos_v) || (a < pos_k && pk[a] >= pv[b]);
      if (take_k) { order_kind[n_order] = 0; order_idx[n_order++] = ik[a]; sel_k[nk++] = ik[a++]; }
      else        { order_kind[n_order] = 1; order_idx[n_order++] = iv[b]; sel_v[nv++] = iv[b++]; }
    }
  } else {
    const int kb = min(sp.k_budget, pos_k), vb = min(sp.v_budget, pos_v);
    for (int i = 0; i < kb; ++i) { order_kind[n_order] = 0; order_idx[n_order++] = ik[i]; sel_k[nk++] = ik[i]; }
    for (int i = 0; i < vb; ++i) { order_kind[n_order] = 1; order_idx[n_order++] = iv[i]; sel_v[nv++] = iv[i]; }
  }
}

// One wave per page job.  Lane l handles token t = l / NG, quant group g = l % NG.
// MODE 0: write base + metadata + counts.  MODE 1: write residual slots.
template <int D, int BITS, int MODE>
__global__ __launch_bounds__(256) void store_pages_kernel(carekv_arena A, carekv_store_params sp,
                                                          const uint16_t* __restrict__ Kx,
                                                          const uint16_t* __restrict__ Vx,
                                                          const carekv_page_job* __restrict__ jobs,
                                                          int n_jobs, StoreWs ws) {
  constexpr int NG = D / 32;       // quant groups == K channel groups
  constexpr int RB = row_bytes(D, BITS);
  constexpr int CB = 4 * BITS;     // packed bytes per 32 codes
  const int lane = threadIdx.x & 63;
  const int job_id = blockIdx.x * 4 + (threadIdx.x >> 6);
  // the call's slot-overflow word (after the job records) starts clear in
  // the count pass; the write pass sets it
  if (MODE == 0 && blockIdx.x == 0 && threadIdx.x == 0) ws.v[n_jobs * 4] = 0;
  if (job_id >= n_jobs) return;
  const carekv_page_job job = jobs[job_id];
  const int t = lane / NG, g = lane % NG;
  const bool active = t < kPage;
  const int nvld = job.num_valid;
  const long pg = ((long)job.kv_head * A.n_seq + job.seq) * A.max_pages + job.page;
  // a packed KIVI arena's call runs once over the packed prefix and once
  // over a view of its fp16 tail: each launch takes only its own pages
  if (A.kivi_packed && job.page >= A.n_packed[job.seq]) return;
  if (!code_pg_in(A, pg)) return;

  // ---- quantize own (t, g) group of K and V, fp16 chain (or, for the fp16
  // side-buffer base, take the given K_hat / V_hat)
  float xk[32], xv[32], rk[32], rv[32];
  int ck[32], cv[32];
  _Float16 sk = 0, sv = 0;
  float hk[32], hv[32];  // K_hat / V_hat of the fp16 base
  if constexpr (BITS == 16) {
    if (active) {
      const long o = ((long)job_id * kPage + t) * D + g * 32;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        xk[i] = h2f(Kx[o + i]); xv[i] = h2f(Vx[o + i]);
        hk[i] = h2f(sp.k_hat[o + i]); hv[i] = h2f(sp.v_hat[o + i]);
        // residual against the given K_hat (residual_store.py:272-285)
        rk[i] = (t < nvld) ? (float)(_Float16)(xk[i] - hk[i]) : 0.f;
        rv[i] = (t < nvld) ? (float)(_Float16)(xv[i] - hv[i]) : 0.f;
        ck[i] = cv[i] = 0;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) { rk[i] = rv[i] = hk[i] = hv[i] = 0.f; ck[i] = cv[i] = 0; }
    }
  } else if (active) {
    const uint16_t* kp = Kx + ((long)job_id * kPage + t) * D + g * 32;
    const uint16_t* vp = Vx + ((long)job_id * kPage + t) * D + g * 32;
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
      uint4 a = *reinterpret_cast<const uint4*>(kp + i);
      uint4 b = *reinterpret_cast<const uint4*>(vp + i);
      const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xk[i + 2 * j] = h2f((uint16_t)wa[j]); xk[i + 2 * j + 1] = h2f((uint16_t)(wa[j] >> 16));
        xv[i + 2 * j] = h2f((uint16_t)wb[j]); xv[i + 2 * j + 1] = h2f((uint16_t)(wb[j] >> 16));
      }
    }
    if (A.kivi_packed) {
      // packed KIVI prefix page: the caller's 2-bit codes and per-token V
      // scales; the residuals are taken against K_hat / V_hat, which
      // half(code * scale) reproduces (K's per-channel scales live in kchan)
      const long ri = (long)job_id * kPage + t;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        ck[i] = sp.k_codes_in[ri * D + g * 32 + i];
        cv[i] = sp.v_codes_in[ri * D + g * 32 + i];
        hk[i] = h2f(sp.k_hat[ri * D + g * 32 + i]);
        hv[i] = h2f(sp.v_hat[ri * D + g * 32 + i]);
      }
      sv = bits2half(sp.v_scale_in[ri * NG + g]);
    } else if (sp.k_codes_in) {
      // process_page on a page write_base wrote: the caller's base codes and
      // fp16 group scales (residual_store.py:276-285); the page keeps its base
      const long ri = (long)job_id * kPage + t;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        ck[i] = sp.k_codes_in[ri * D + g * 32 + i];
        cv[i] = sp.v_codes_in[ri * D + g * 32 + i];
      }
      sk = bits2half(sp.k_scale_in[ri * NG + g]);
      sv = bits2half(sp.v_scale_in[ri * NG + g]);
    } else if (sp.keep_base) {
      // streaming store of a page the decode appends filled: the page keeps
      // its base, the residual is taken against it as the decode reads it,
      // half(code * half(scale code * master)) (layer.py:1104-1133)
      const long row = pg * kPage + t;
      uint32_t w[BITS];
      load_bytes<CB>(w, A.kcodes + row * RB + g * CB);
#pragma unroll
      for (int i = 0; i < 32; ++i) ck[i] = get_code<BITS>(w, i);
      load_bytes<CB>(w, A.vcodes + row * RB + g * CB);
#pragma unroll
      for (int i = 0; i < 32; ++i) cv[i] = get_code<BITS>(w, i);
      if (A.scale_mode == 1) {
        sk = (_Float16)((float)((const int8_t*)A.kscale)[row * NG + g] * h2f(A.kmaster[pg]));
        sv = (_Float16)((float)((const int8_t*)A.vscale)[row * NG + g] * h2f(A.vmaster[pg]));
      } else {
        sk = bits2half(((const uint16_t*)A.kscale)[row * NG + g]);
        sv = bits2half(((const uint16_t*)A.vscale)[row * NG + g]);
      }
    } else {
      sk = quant_group<BITS>(xk, ck);
      sv = quant_group<BITS>(xv, cv);
    }
    // residual against the fp16 scale (residual_store.py:276-285), or
    // against the KIVI K_hat / V_hat
    const bool kv = A.kivi_packed != 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float bk = kv ? hk[i] : (float)dq(ck[i], sk), bv = kv ? hv[i] : (float)dq(cv[i], sv);
      rk[i] = (t < nvld) ? (float)(_Float16)(xk[i] - bk) : 0.f;
      rv[i] = (t < nvld) ? (float)(_Float16)(xv[i] - bv) : 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) { rk[i] = rv[i] = 0.f; ck[i] = cv[i] = 0; }
  }

  // ---- candidate errors (fp32): K per channel group, V per 4-token block
  float sq_k = 0.f, sq_v = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) { sq_k += rk[i] * rk[i]; sq_v += rv[i] * rv[i]; }
  float nrm_k = active ? sqrtf(sq_k) : 0.f;      // ||R_K[t, cg]||
  float kerr[NG], verr[kVtb];
  {
    float s = nrm_k;  // sum over tokens (lanes with equal g)
#pragma unroll
    for (int o = NG; o < NG * kPage; o <<= 1) s += __shfl_xor(s, o, 64);
#pragma unroll
    for (int c = 0; c < NG; ++c) {
      const float sc = __shfl(s, c, 64);
      kerr[c] = nvld > 0 ? sc / (float)nvld : 0.f;
    }
    float tv = sq_v;  // ||R_V[t]||^2 over the row: sum over the NG lanes of token t
#pragma unroll
    for (int o = 1; o < NG; o <<= 1) tv += __shfl_xor(tv, o, 64);
    const float tn = (active && t < nvld) ? sqrtf(tv) : 0.f;
#pragma unroll
    for (int b = 0; b < kVtb; ++b) {
      float acc = 0.f;
      for (int i = 0; i < kVtb; ++i) acc += __shfl(tn, (b * kVtb + i) * NG, 64);
      const int t0 = b * kVtb, t1 = min(t0 + kVtb, nvld);
      verr[b] = t1 > t0 ? acc / (float)(t1 - t0) : 0.f;
    }
  }
  double struct_prior = 1.0;
  if (job.is_recent) struct_prior *= 1.5;
  if (job.token_start < sp.sink_tokens) struct_prior *= 2.0;
  int sel_k[NG], sel_v[kVtb], okind[NG + kVtb], oidx[NG + kVtb], nk, nv, nord;
  select_candidates<NG>(kerr, verr, sp, struct_prior, sel_k, nk, sel_v, nv, okind, oidx, nord);

  if constexpr (MODE == 0 && BITS == 16) {
    // ---- fp16 side-buffer rows (cache.py:800-818) and sum of V_hat^2; on a
    // code-page map only the pages it holds (the host sends no others)
    if (active && code_pg_in(A, pg)) {
      uint32_t wk[16], wv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        wk[i] = (uint32_t)f2h(hk[2 * i]) | ((uint32_t)f2h(hk[2 * i + 1]) << 16);
        wv[i] = (uint32_t)f2h(hv[2 * i]) | ((uint32_t)f2h(hv[2 * i + 1]) << 16);
      }
      const long cpg = code_pg(A, pg);
      store_bytes<64>(A.kcodes + (cpg * kPage + t) * RB + g * 64, wk);
      store_bytes<64>(A.vcodes + (cpg * kPage + t) * RB + g * 64, wv);
    }
    float vs = 0.f;
    if (active && t < nvld) {
#pragma unroll
      for (int i = 0; i < 32; ++i) vs += hv[i] * hv[i];
    }
    vs = wave_sum(vs);
    if (lane == 0) A.v_sq[pg] = vs;
  }
  if (MODE == 0 && BITS != 16 && !A.kivi_packed && (sp.keep_base || sp.k_codes_in)) {
    // ---- the page keeps its base; only the sum of V_hat^2 is refreshed, over
    // the rows as the decode reads them back
    float vs = 0.f;
    if (active && t < nvld) {
      _Float16 svr = sv;
      if (sp.k_codes_in) {
        const long row = pg * kPage + t;
        svr = A.scale_mode == 1 ? (_Float16)((float)((const int8_t*)A.vscale)[row * NG + g] * h2f(A.vmaster[pg]))
                                : bits2half(((const uint16_t*)A.vscale)[row * NG + g]);
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) { const float vh = (float)dq(cv[i], svr); vs += vh * vh; }
    }
    vs = wave_sum(vs);
    if (lane == 0) A.v_sq[pg] = vs;
  } else if constexpr (MODE == 0 && BITS != 16) {
    // ---- packed base codes
    if (active) {
      uint32_t w[BITS];
      pack_group<BITS>(ck, w);
      store_bytes<CB>(A.kcodes + (pg * kPage + t) * RB + g * CB, w);
      pack_group<BITS>(cv, w);
      store_bytes<CB>(A.vcodes + (pg * kPage + t) * RB + g * CB, w);
    }
    // ---- scales
    if (A.scale_mode == 1) {
      const float mk = wave_max(active ? (float)sk : 0.f);
      const float mv = wave_max(active ? (float)sv : 0.f);
      const _Float16 mkh = (_Float16)(mk / 127.f), mvh = (_Float16)(mv / 127.f);
      const int8_t qk = scale_code((float)sk, (float)mkh), qv = scale_code((float)sv, (float)mvh);
      if (active) {
        ((int8_t*)A.kscale)[(pg * kPage + t) * NG + g] = qk;
        ((int8_t*)A.vscale)[(pg * kPage + t) * NG + g] = qv;
      }
      // V_hat as read back from the cache: half(code * half(scode * master))
      const _Float16 svr = (_Float16)((float)qv * (float)mvh);
      float vs = 0.f;
      if (active && t < nvld) {
#pragma unroll
        for (int i = 0; i < 32; ++i) { const float vh = (float)dq(cv[i], svr); vs += vh * vh; }
      }
      vs = wave_sum(vs);
      if (lane == 0) {
        A.kmaster[pg] = half2bits(mkh);
        A.vmaster[pg] = half2bits(mvh);
        A.v_sq[pg] = vs;
      }
    } else {
      if (active) {
        ((uint16_t*)A.kscale)[(pg * kPage + t) * NG + g] = half2bits(sk);
        ((uint16_t*)A.vscale)[(pg * kPage + t) * NG + g] = half2bits(sv);
      }
      float vs = 0.f;
      if (active && t < nvld) {
#pragma unroll
        for (int i = 0; i < 32; ++i) { const float vh = (float)dq(cv[i], sv); vs += vh * vh; }
      }
      vs = wave_sum(vs);
      if (lane == 0) A.v_sq[pg] = vs;
    }
  }
  if (MODE == 0) {
    // ---- K sketch: half(mean_t R_K[t, cg] @ P)  (residual_store.py:305,311-312)
    {
      float mean[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        float s = rk[i];
#pragma unroll
        for (int o = NG; o < NG * kPage; o <<= 1) s += __shfl_xor(s, o, 64);
        mean[i] = nvld > 0 ? s / (float)nvld : 0.f;
      }
      const int SD = A.sketch_dim;
      for (int k = t; k < SD; k += kPage) {
        if (!active) break;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < 32; ++c) acc += mean[c] * sp.sketch_proj[c * SD + k];
        A.k_sketch[(pg * NG + g) * SD + k] = f2h(acc);
      }
    }
    if (lane < NG) A.k_err[pg * NG + lane] = f2h(kerr[lane]);
    if (lane < kVtb) A.v_err[pg * kVtb + lane] = f2h(verr[lane]);
    // streaming store: the slot ids the page holds from an earlier store (a
    // prompt's partial last page) are reused first, so only the rest are
    // counted for new ids; a page without metadata holds none (its slot
    // tables are cleared here, before the write pass reads them)
    int reuse_k = 0, reuse_v = 0;
    if (sp.reuse_slots) {
      if (A.has_meta[pg]) {
#pragma unroll
        for (int c = 0; c < NG; ++c) reuse_k += A.k_slot[pg * NG + c] >= 0;
#pragma unroll
        for (int b = 0; b < kVtb; ++b) reuse_v += A.v_slot[pg * kVtb + b] >= 0;
      } else {
        if (lane < NG) A.k_slot[pg * NG + lane] = -1;
        if (lane < kVtb) A.v_slot[pg * kVtb + lane] = -1;
      }
    }
    if (lane == 0) {
      A.valid[pg] = nvld;
      A.has_meta[pg] = 1;
      ws.v[job_id * 4 + 0] = nk - min(reuse_k, nk);
      ws.v[job_id * 4 + 1] = nv - min(reuse_v, nv);
    }
  } else {
    // ---- residual slots at the scanned bases (residual_store.py:424-438)
    const int base_k = ws.v[job_id * 4 + 2], base_v = ws.v[job_id * 4 + 3];
    const long seq_off = (long)job.seq * A.n_slots;
    constexpr int KSB = kPage * 32 / 2;     // 16 tokens x 32 channels, 4-bit
    const int VSB = kVtb * D / 2;
    int kslot_of[NG], vslot_of[kVtb];
#pragma unroll
    for (int c = 0; c < NG; ++c) kslot_of[c] = -1;
#pragma unroll
    for (int b = 0; b < kVtb; ++b) vslot_of[b] = -1;
    // streaming store: the page's earlier slot ids, ascending, go to the
    // first selected candidates of their kind (the count pass left them out
    // of the new ids; a page without metadata had its tables cleared there)
    int old_k[NG], old_v[kVtb], n_ok = 0, n_ov = 0;
    if (sp.reuse_slots) {
#pragma unroll
      for (int c = 0; c < NG; ++c) {
        const int id = A.k_slot[pg * NG + c];
        if (id >= 0) old_k[n_ok++] = id;
      }
#pragma unroll
      for (int b = 0; b < kVtb; ++b) {
        const int id = A.v_slot[pg * kVtb + b];
        if (id >= 0) old_v[n_ov++] = id;
      }
      for (int i = 1; i < n_ok; ++i)
        for (int j = i; j > 0 && old_k[j] < old_k[j - 1]; --j) { const int u = old_k[j]; old_k[j] = old_k[j - 1]; old_k[j - 1] = u; }
      for (int i = 1; i < n_ov; ++i)
        for (int j = i; j > 0 && old_v[j] < old_v[j - 1]; --j) { const int u = old_v[j]; old_v[j] = old_v[j - 1]; old_v[j - 1] = u; }
    }
    // new slot ids past the arena are dropped (never written) and flagged
    for (int i = 0; i < nk; ++i) {
      if (i < n_ok) kslot_of[sel_k[i]] = old_k[i];
      else if (base_k + (i - n_ok) < A.n_slots) kslot_of[sel_k[i]] = base_k + (i - n_ok);
      else if (lane == 0) ws.v[n_jobs * 4] = 1;
    }
    for (int i = 0; i < nv; ++i) {
      if (i < n_ov) vslot_of[sel_v[i]] = old_v[i];
      else if (base_v + (i - n_ov) < A.n_slots) vslot_of[sel_v[i]] = base_v + (i - n_ov);
      else if (lane == 0) ws.v[n_jobs * 4] = 1;
    }
    // K payload of channel group g: pack_4bit(R_K[:, cg]) over all 16 rows
    {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(rk[i]));
#pragma unroll
      for (int o = NG; o < NG * kPage; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      const float s = fmaxf(m, 1e-8f) / 7.0f;
      const int slot = kslot_of[g];
      if (active && slot >= 0) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int c = (int)fminf(fmaxf(rintf(rk[i] / s), -8.f), 7.f);
          w[i >> 3] |= ((uint32_t)c & 15u) << (4 * (i & 7));
        }
        int8_t* dst = A.k_res + (seq_off + slot) * KSB + t * 16;
        *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        if (t == 0) A.k_res_scale[seq_off + slot] = f2h(s);
      }
    }
    // V payload of block t/4: pack_4bit(R_V[4b..4b+3, :])
    {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(rv[i]));
#pragma unroll
      for (int o = 1; o < NG * kVtb; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      const float s = fmaxf(m, 1e-8f) / 7.0f;
      const int b = t / kVtb;
      const int slot = active ? vslot_of[b] : -1;
      if (slot >= 0) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int c = (int)fminf(fmaxf(rintf(rv[i] / s), -8.f), 7.f);
          w[i >> 3] |= ((uint32_t)c & 15u) << (4 * (i & 7));
        }
        int8_t* dst = A.v_res + (seq_off + slot) * VSB + (t - b * kVtb) * (D / 2) + g * 16;
        *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        if (t == b * kVtb && g == 0) A.v_res_scale[seq_off + slot] = f2h(s);
      }
    }
    if (lane < NG) A.k_slot[pg * NG + lane] = kslot_of[lane];
    if (lane < kVtb) A.v_slot[pg * kVtb + lane] = vslot_of[lane];
  }
}

// Exclusive scan of per-job slot counts inside each sequence group (jobs of
// one group are contiguous and ordered like the reference's process_page
// calls); bases start at next_slot[seq], which is advanced.
__global__ __launch_bounds__(256) void store_scan_kernel(carekv_arena A, const carekv_page_job* __restrict__ jobs,
                                                         const int32_t* __restrict__ group_ptr, StoreWs ws) {
  // chunks of 1024 jobs: 4 consecutive jobs a thread, a wave scan of the
  // thread totals (shuffles), the 4 wave totals through LDS
  __shared__ int s_wk[4], s_wv[4];
  __shared__ int carry_k, carry_v;
  const int g = blockIdx.x;
  const int j0 = group_ptr[g], j1 = group_ptr[g + 1];
  if (j1 <= j0) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int seq = jobs[j0].seq;
  if (threadIdx.x == 0) { carry_k = A.next_slot[2 * seq]; carry_v = A.next_slot[2 * seq + 1]; }
  __syncthreads();
  for (int base = j0; base < j1; base += 1024) {
    const int jb = base + 4 * threadIdx.x;
    int ck[4], cv[4], tk = 0, tv = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = jb + i < j1;
      ck[i] = ok ? ws.v[(jb + i) * 4] : 0;
      cv[i] = ok ? ws.v[(jb + i) * 4 + 1] : 0;
      tk += ck[i];
      tv += cv[i];
    }
    int ik = tk, iv = tv;  // inclusive scan of the thread totals over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int yk = __shfl_up(ik, o, 64), yv = __shfl_up(iv, o, 64);
      if (lane >= o) { ik += yk; iv += yv; }
    }
    if (lane == 63) { s_wk[w] = ik; s_wv[w] = iv; }
    __syncthreads();
    int off_k = carry_k, off_v = carry_v;  // slots before this thread's first job
    for (int ww = 0; ww < w; ++ww) { off_k += s_wk[ww]; off_v += s_wv[ww]; }
    off_k += ik - tk;
    off_v += iv - tv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (jb + i < j1) {
        ws.v[(jb + i) * 4 + 2] = off_k;
        ws.v[(jb + i) * 4 + 3] = off_v;
      }
      off_k += ck[i];
      off_v += cv[i];
    }
    __syncthreads();  // every thread has read the carries and wave totals
    if (threadIdx.x == 0) {
      carry_k += ((s_wk[0] + s_wk[1]) + s_wk[2]) + s_wk[3];
      carry_v += ((s_wv[0] + s_wv[1]) + s_wv[2]) + s_wv[3];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) { A.next_slot[2 * seq] = carry_k; A.next_slot[2 * seq + 1] = carry_v; }
}

// KIVI-style value (kivi_helpers.py:35-59): half(clamp(rint(half(x / s))) * s)
// in fp16 arithmetic; a NaN quotient (0/0) stays NaN through rint and
// clamp, as torch's clamp propagates it.
__device__ __forceinline__ float kivi_value(float x, float scale, int bits) {
  const float qmax = (float)((1 << (bits - 1)) - 1);
  const float q = rintf((float)(_Float16)(x / scale));
  const float c = (q != q) ? q : fminf(fmaxf(q, -qmax - 1.f), qmax);
  // the product's sign is the code's (scale >= 0): a code of -0 (the rint of
  // a small negative quotient) gives -0 as in the reference, which a fused
  // multiply-add with a +0 addend would turn into +0
  const float r = (float)(_Float16)(c * scale);
  return (c != c) ? r : copysignf(r, c);
}
// scale = half(max|x| / qmax); the 1e-8 floor is 0 in fp16 (a no-op)
__device__ __forceinline__ float kivi_scale(float amax, int bits) {
  return (float)(_Float16)(amax / (float)((1 << (bits - 1)) - 1));
}

// quant_dequant_kivi_k: one work-group per (matrix, 64 columns); 4 row
// groups reduce max|x| per column through LDS.
__global__ __launch_bounds__(256) void kivi_channel_kernel(const uint16_t* __restrict__ x, int rows, int D, int bits,
                                                           uint16_t* __restrict__ out) {
  __shared__ float s_max[4][64];
  const int m = blockIdx.x, c0 = blockIdx.y * 64;
  const int lane = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int d = c0 + lane;
  const long base = (long)m * rows * D;
  float a = 0.f;
  if (d < D)
    for (int r = rg; r < rows; r += 4) a = fmaxf(a, fabsf(h2f(x[base + (long)r * D + d])));
  s_max[rg][lane] = a;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_max[0][lane], s_max[1][lane]), fmaxf(s_max[2][lane], s_max[3][lane]));
  const float sc = kivi_scale(amax, bits);
  if (d < D)
    for (int r = rg; r < rows; r += 4) {
      const long i = base + (long)r * D + d;
      out[i] = f2h(kivi_value(h2f(x[i]), sc, bits));
    }
}

// quant_dequant_kivi_v: one wave per row.
__global__ __launch_bounds__(256) void kivi_token_kernel(const uint16_t* __restrict__ x, long n_rows, int D, int bits,
                                                         uint16_t* __restrict__ out) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;
  const uint16_t* xr = x + row * D;
  float a = 0.f;
  for (int d = lane; d < D; d += 64) a = fmaxf(a, fabsf(h2f(xr[d])));
  const float sc = kivi_scale(wave_max(a), bits);
  for (int d = lane; d < D; d += 64) out[row * D + d] = f2h(kivi_value(h2f(xr[d]), sc, bits));
}

// Decode append for the fp16 side-buffer base: one wave per row; K per
// channel over the one row (scale |k_d| / qmax), V per token
// (layer.py:1037-1075, cache.py:820-838).
template <int D>
__global__ __launch_bounds__(256) void append_hat_rows_kernel(carekv_arena A, const uint16_t* __restrict__ Kx,
                                                              const uint16_t* __restrict__ Vx,
                                                              const int32_t* __restrict__ dest, int n_rows) {
  constexpr int NG = D / 32;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int seq = dest[row * 4], kvh = dest[row * 4 + 1], page = dest[row * 4 + 2], fresh = dest[row * 4 + 3];
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int off = fresh ? 0 : A.valid[pg];
  if (off >= kPage) return;  // caller contract violated; never write past the page
  if (!code_pg_in(A, pg)) return;  // a page the code-page map does not hold: never written
  const long cpg = code_pg(A, pg);
  uint16_t* krow = reinterpret_cast<uint16_t*>(A.kcodes) + (cpg * kPage + off) * D;
  uint16_t* vrow = reinterpret_cast<uint16_t*>(A.vcodes) + (cpg * kPage + off) * D;
  float av = 0.f;
  for (int d = lane; d < D; d += 64) av = fmaxf(av, fabsf(h2f(Vx[(long)row * D + d])));
  const float sv = kivi_scale(wave_max(av), A.hat_bits_v);
  float vs = 0.f;  // this row's share of the page's sum of V_hat^2
  for (int d = lane; d < D; d += 64) {
    const float k = h2f(Kx[(long)row * D + d]);
    krow[d] = f2h(kivi_value(k, kivi_scale(fabsf(k), A.hat_bits_k), A.hat_bits_k));
    const uint16_t vh = f2h(kivi_value(h2f(Vx[(long)row * D + d]), sv, A.hat_bits_v));
    vrow[d] = vh;
    vs += h2f(vh) * h2f(vh);
  }
  vs = wave_sum(vs);
  // the store on fill, unless the caller's streaming store writes the page's
  // metadata (it reads the slots the page holds)
  const bool full = off + 1 == kPage && !A.streaming_store;
  if (lane == 0) {
    A.valid[pg] = off + 1;
    if (fresh) A.has_meta[pg] = full ? 1 : 0;
    if (full) A.has_meta[pg] = 1;
    A.v_sq[pg] = full ? 0.f : (fresh ? 0.f : A.v_sq[pg]) + vs;
  }
  if (full) {
    // store on page fill with K_orig = K_hat: zero residual -> no slots,
    // zero errors, zero sketch (layer.py:1088-1101)
    if (lane < NG) { A.k_slot[pg * NG + lane] = -1; A.k_err[pg * NG + lane] = 0; }
    if (lane < kVtb) { A.v_slot[pg * kVtb + lane] = -1; A.v_err[pg * kVtb + lane] = 0; }
    for (int i = lane; i < NG * A.sketch_dim; i += 64) A.k_sketch[pg * NG * A.sketch_dim + i] = 0;
  }
}

// Decode append: one wave per (row); lane g < D/32 quantizes group g.
// Int8 page scales (scale_mode 1) take one of two encodings:
//   * the reference's (cache.py:689-695): the row's scale codes against the
//     page's fixed master, clamped at 1e-8 -- a page the decode opens keeps
//     master 0, so its rows read back as zero;
//   * rescale_open: the page is encoded as write_base encodes a page holding
//     its valid rows (cache.py:592-604): master = half(max scale / 127) over
//     the rows so far and every row's code against it, from the fp16 scales
//     of the open page kept in open_kscale / open_vscale (this row's are
//     added there).  When the page fills, its bytes are those write_base
//     gives the 16 rows.  A page that holds stored residual slots (a
//     prompt's partial last page) is not re-encoded: its slots are residuals
//     against its rows as the prompt wrote them, so it keeps the reference's
//     fixed-master encoding (the first form) until it fills.
// The page's sum of V_hat^2 (v_sq, read by the query-aware K score of its
// stored K slots) is recomputed over the valid rows as they now read back.
// Coded rows (append_to_page, cache.py:656-701): the caller's int8 codes and
// fp16 group scales replace the row quantizer, and a full page gets no
// metadata (the store on fill belongs to the decode step, not the append).
struct CodedRows {
  const int8_t* kc;
  const uint16_t* ks;
  const int8_t* vc;
  const uint16_t* vs;
};

template <int D, int BITS>
__global__ __launch_bounds__(256) void append_rows_kernel(carekv_arena A, const uint16_t* __restrict__ Kx,
                                                          const uint16_t* __restrict__ Vx,
                                                          const int32_t* __restrict__ dest, int n_rows,
                                                          CodedRows cr) {
  constexpr int NG = D / 32;
  constexpr int RB = row_bytes(D, BITS);
  constexpr int CB = 4 * BITS;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int seq = dest[row * 4], kvh = dest[row * 4 + 1], page = dest[row * 4 + 2], fresh = dest[row * 4 + 3];
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int off = fresh ? 0 : A.valid[pg];
  if (off >= kPage) return;  // caller contract violated; never write past the page
  const bool i8 = A.scale_mode == 1;
  // stored slots on the page (only a page with metadata can hold any)
  bool slots = false;
  if (!fresh && A.has_meta[pg]) {
    const int id = lane < NG ? A.k_slot[pg * NG + lane]
                             : (lane < NG + kVtb ? A.v_slot[pg * kVtb + lane - NG] : -1);
    slots = __ballot(id >= 0) != 0ull;
  }
  const bool rescale = i8 && A.rescale_open != 0 && !slots;
  int cv[32];
  _Float16 sk = (_Float16)0.f, sv = (_Float16)0.f;
  if (lane < NG) {
    const int g = lane;
    float xk[32], xv[32];
    int ck[32];
    if (cr.kc) {
      for (int i = 0; i < 32; ++i) {
        ck[i] = cr.kc[(long)row * D + g * 32 + i];
        cv[i] = cr.vc[(long)row * D + g * 32 + i];
      }
      sk = bits2half(cr.ks[(long)row * NG + g]);
      sv = bits2half(cr.vs[(long)row * NG + g]);
    } else {
      for (int i = 0; i < 32; ++i) {
        xk[i] = h2f(Kx[(long)row * D + g * 32 + i]);
        xv[i] = h2f(Vx[(long)row * D + g * 32 + i]);
      }
      sk = quant_group<BITS>(xk, ck);
      sv = quant_group<BITS>(xv, cv);
    }
    uint32_t w[BITS];
    pack_group<BITS>(ck, w);
    store_bytes<CB>(A.kcodes + (pg * kPage + off) * RB + g * CB, w);
    pack_group<BITS>(cv, w);
    store_bytes<CB>(A.vcodes + (pg * kPage + off) * RB + g * CB, w);
    if (!i8) {
      ((uint16_t*)A.kscale)[(pg * kPage + off) * NG + g] = half2bits(sk);
      ((uint16_t*)A.vscale)[(pg * kPage + off) * NG + g] = half2bits(sv);
    }
  }
  // lane l < 16 NG: row r = l / NG, group gg = l % NG of the page
  const int r = lane / NG, gg = lane % NG;
  const bool cell = lane < kPage * NG && r <= off;
  float mk = 0.f, mv = 0.f;  // the page's masters after this row (int8 scales)
  if (rescale) {
    const long ob = ((long)kvh * A.n_seq + seq) * kPage * NG;
    const float nk = __shfl((float)sk, gg, 64), nv = __shfl((float)sv, gg, 64);
    float s_k = 0.f, s_v = 0.f;
    if (cell) {
      s_k = r < off ? h2f(A.open_kscale[ob + r * NG + gg]) : nk;
      s_v = r < off ? h2f(A.open_vscale[ob + r * NG + gg]) : nv;
    }
    mk = (float)(_Float16)(wave_max(s_k) / 127.f);
    mv = (float)(_Float16)(wave_max(s_v) / 127.f);
    if (cell) {
      ((int8_t*)A.kscale)[(pg * kPage + r) * NG + gg] = scale_code(s_k, mk);
      ((int8_t*)A.vscale)[(pg * kPage + r) * NG + gg] = scale_code(s_v, mv);
    }
    if (lane < NG) {
      A.open_kscale[ob + off * NG + lane] = half2bits(sk);
      A.open_vscale[ob + off * NG + lane] = half2bits(sv);
    }
  } else if (i8) {
    mk = fmaxf(fresh ? 0.f : h2f(A.kmaster[pg]), 1e-8f);
    mv = fmaxf(fresh ? 0.f : h2f(A.vmaster[pg]), 1e-8f);
    if (lane < NG) {
      ((int8_t*)A.kscale)[(pg * kPage + off) * NG + lane] = scale_code((float)sk, mk);
      ((int8_t*)A.vscale)[(pg * kPage + off) * NG + lane] = scale_code((float)sv, mv);
    }
  }
  // sum of V_hat^2 over the valid rows: earlier rows from the page, this row
  // from the registers of lanes g < NG
  float vs = 0.f;
  if (lane < NG) {
    _Float16 s = sv;
    if (i8) s = (_Float16)((float)scale_code((float)sv, mv) * (rescale ? mv : (fresh ? 0.f : h2f(A.vmaster[pg]))));
#pragma unroll
    for (int i = 0; i < 32; ++i) { const float x = (float)dq(cv[i], s); vs += x * x; }
  }
  if (cell && r < off) {
    uint32_t w[BITS];
    load_bytes<CB>(w, A.vcodes + (pg * kPage + r) * RB + gg * CB);
    _Float16 s;
    if (i8) {
      const int8_t q = ((const int8_t*)A.vscale)[(pg * kPage + r) * NG + gg];
      s = (_Float16)((float)(rescale ? scale_code(h2f(A.open_vscale[((long)kvh * A.n_seq + seq) * kPage * NG +
                                                                    r * NG + gg]), mv) : q) *
                     (rescale ? mv : h2f(A.vmaster[pg])));
    } else {
      s = bits2half(((const uint16_t*)A.vscale)[(pg * kPage + r) * NG + gg]);
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) { const float x = (float)dq(get_code<BITS>(w, i), s); vs += x * x; }
  }
  vs = wave_sum(vs);
  // the decode step's store on fill, unless the caller's streaming store
  // writes the page's metadata (it reads the slots the page holds)
  const bool full = off + 1 == kPage && !cr.kc && !A.streaming_store;
  if (lane == 0) {
    A.valid[pg] = off + 1;
    if (rescale) { A.kmaster[pg] = half2bits((_Float16)mk); A.vmaster[pg] = half2bits((_Float16)mv); }
    else if (fresh && i8) { A.kmaster[pg] = 0; A.vmaster[pg] = 0; }
    if (fresh) A.has_meta[pg] = full ? 1 : 0;
    if (full) A.has_meta[pg] = 1;
    A.v_sq[pg] = full ? 0.f : vs;
  }
  if (full) {
    // store on page fill with K_orig = K_hat: zero residual -> no slots,
    // zero errors, zero sketch (layer.py:1088-1146)
    if (lane < NG) { A.k_slot[pg * NG + lane] = -1; A.k_err[pg * NG + lane] = 0; }
    if (lane < kVtb) { A.v_slot[pg * kVtb + lane] = -1; A.v_err[pg * kVtb + lane] = 0; }
    for (int i = lane; i < NG * A.sketch_dim; i += 64) A.k_sketch[pg * NG * A.sketch_dim + i] = 0;
  }
}

// read_base_concat for one (seq, kv head): unpacked codes + fp16 scales.
template <int D, int BITS>
__global__ __launch_bounds__(256) void read_pages_kernel(carekv_arena A, int seq, int kvh, int n_pages,
                                                         const int32_t* __restrict__ page_ids,
                                                         const int32_t* __restrict__ row_start, int8_t* kc,
                                                         uint16_t* ks, int8_t* vc, uint16_t* vs) {
  constexpr int NG = D / 32;
  constexpr int RB = row_bytes(D, BITS);
  constexpr int CB = 4 * BITS;
  const int p = blockIdx.x;
  if (p >= n_pages) return;
  const int page = page_ids ? page_ids[p] : p;
  if (page < 0 || page >= A.max_pages) return;
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int n = A.valid[pg];
  const int r0 = row_start[p];
  for (int idx = threadIdx.x; idx < n * NG; idx += blockDim.x) {
    const int t = idx / NG, g = idx % NG;
    const long out_row = r0 + t;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      const int8_t* src = (which ? A.vcodes : A.kcodes) + (pg * kPage + t) * RB + g * CB;
      uint32_t w[BITS];
      load_bytes<CB>(w, src);
      int8_t* dst = (which ? vc : kc) + out_row * D + g * 32;
      for (int i = 0; i < 32; ++i) dst[i] = (int8_t)get_code<BITS>(w, i);
      uint16_t s;
      if (A.scale_mode == 1) {
        const int8_t q = ((const int8_t*)(which ? A.vscale : A.kscale))[(pg * kPage + t) * NG + g];
        const uint16_t m = which ? A.vmaster[pg] : A.kmaster[pg];
        s = f2h((float)q * h2f(m));
      } else {
        s = ((const uint16_t*)(which ? A.vscale : A.kscale))[(pg * kPage + t) * NG + g];
      }
      (which ? vs : ks)[out_row * NG + g] = s;
    }
  }
}

// Codes and scales of the KIVI quant-dequant (carekv_kivi_codes): one
// work-group per (matrix, 64 columns) for K per channel over the rows, one
// wave per row for V per token.  A scale whose max|x| is 0 is stored as NaN.
__device__ __forceinline__ int kivi_code(float x, float scale, int bits) {
  const float qmax = (float)((1 << (bits - 1)) - 1);
  const float q = rintf((float)(_Float16)(x / scale));
  return (q != q) ? 0 : (int)fminf(fmaxf(q, -qmax - 1.f), qmax);
}
__global__ __launch_bounds__(256) void kivi_channel_codes_kernel(const uint16_t* __restrict__ x, int rows, int D,
                                                                 int bits, int8_t* __restrict__ codes,
                                                                 uint16_t* __restrict__ scale) {
  __shared__ float s_max[4][64];
  const int m = blockIdx.x, c0 = blockIdx.y * 64;
  const int lane = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int d = c0 + lane;
  const long base = (long)m * rows * D;
  float a = 0.f;
  if (d < D)
    for (int r = rg; r < rows; r += 4) a = fmaxf(a, fabsf(h2f(x[base + (long)r * D + d])));
  s_max[rg][lane] = a;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_max[0][lane], s_max[1][lane]), fmaxf(s_max[2][lane], s_max[3][lane]));
  const float sc = kivi_scale(amax, bits);
  if (d < D) {
    for (int r = rg; r < rows; r += 4) {
      const long i = base + (long)r * D + d;
      codes[i] = (int8_t)kivi_code(h2f(x[i]), sc, bits);
    }
    if (rg == 0) scale[(long)m * D + d] = amax == 0.f ? (uint16_t)0x7e00u : f2h(sc);
  }
}
__global__ __launch_bounds__(256) void kivi_token_codes_kernel(const uint16_t* __restrict__ x, long n_rows, int D,
                                                               int bits, int8_t* __restrict__ codes,
                                                               uint16_t* __restrict__ scale) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;
  const uint16_t* xr = x + row * D;
  float a = 0.f;
  for (int d = lane; d < D; d += 64) a = fmaxf(a, fabsf(h2f(xr[d])));
  const float amax = wave_max(a);
  const float sc = kivi_scale(amax, bits);
  for (int d = lane; d < D; d += 64) codes[row * D + d] = (int8_t)kivi_code(h2f(xr[d]), sc, bits);
  if (lane == 0) scale[row] = amax == 0.f ? (uint16_t)0x7e00u : f2h(sc);
}

// read_base_hat_concat (carekv_read_hat_pages): one 64-thread block per page;
// K_hat / V_hat rows of a fp16 page (the side-buffer base, or the tail of a
// packed KIVI arena) copied, of a packed KIVI prefix page dequantised.
template <int D>
__global__ __launch_bounds__(64) void read_hat_pages_kernel(carekv_arena A, int seq, int kvh, int n_pages,
                                                            const int32_t* __restrict__ page_ids,
                                                            const int32_t* __restrict__ row_start,
                                                            uint16_t* __restrict__ kh, uint16_t* __restrict__ vh) {
  constexpr int NG = D / 32;
  constexpr int RB2 = row_bytes(D, 2);
  const int p = blockIdx.x;
  if (p >= n_pages) return;
  const int page = page_ids ? page_ids[p] : p;
  if (page < 0 || page >= A.max_pages) return;
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int n = A.valid[pg];
  const long r0 = row_start[p];
  const bool packed = A.kivi_packed && page < A.n_packed[seq];
  if (packed) {
    const uint16_t* kc = A.kchan + ((long)kvh * A.n_seq + seq) * D;
    for (int idx = threadIdx.x; idx < n * D; idx += 64) {
      const int t = idx / D, d = idx % D, g = d / 32;
      uint32_t w[2];
      load_bytes<8>(w, A.kcodes + (pg * kPage + t) * RB2 + g * 8);
      const int ck = get_code<2>(w, d % 32);
      load_bytes<8>(w, A.vcodes + (pg * kPage + t) * RB2 + g * 8);
      const int cv = get_code<2>(w, d % 32);
      const _Float16 vs = bits2half(((const uint16_t*)A.vscale)[(pg * kPage + t) * NG + g]);
      kh[(r0 + t) * D + d] = half2bits(dq(ck, bits2half(kc[d])));
      vh[(r0 + t) * D + d] = half2bits(dq(cv, vs));
    }
    return;
  }
  const uint16_t* ksrc;
  const uint16_t* vsrc;
  if (A.kivi_packed) {
    const int tp = page - A.n_packed[seq];
    if (tp >= A.tail_pages) return;
    const long tpg = ((long)kvh * A.n_seq + seq) * A.tail_pages + tp;
    ksrc = A.tail_k + tpg * kPage * D;
    vsrc = A.tail_v + tpg * kPage * D;
  } else {
    ksrc = reinterpret_cast<const uint16_t*>(A.kcodes) + pg * kPage * D;
    vsrc = reinterpret_cast<const uint16_t*>(A.vcodes) + pg * kPage * D;
  }
  for (int idx = threadIdx.x; idx < n * D; idx += 64) {
    kh[r0 * D + idx] = ksrc[idx];
    vh[r0 * D + idx] = vsrc[idx];
  }
}

// Row quantizer API (quantizer.py:31-64 + pack_codes_2d).
template <int BITS>
__global__ void quantize_rows_kernel(const uint16_t* __restrict__ x, int rows, int D, int pack, int8_t* codes,
                                     uint16_t* scale) {
  const int G = D / 32;
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * G) return;
  const int r = id / G, g = id % G;
  float v[32];
  int c[32];
  for (int i = 0; i < 32; ++i) v[i] = h2f(x[(long)r * D + g * 32 + i]);
  const _Float16 s = quant_group<BITS>(v, c);
  scale[id] = half2bits(s);
  if (pack) {
    uint32_t w[BITS];
    pack_group<BITS>(c, w);
    int8_t* dst = codes + (long)r * row_bytes(D, BITS) + g * 4 * BITS;
    for (int i = 0; i < 4 * BITS; ++i) dst[i] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
  } else {
    for (int i = 0; i < 32; ++i) codes[(long)r * D + g * 32 + i] = (int8_t)c[i];
  }
}

}  // namespace carekv

// ------------------------------------------------------------------ host side
#include "host_util.h"

using namespace carekv;

// per job 4 int32 (counts, then slot bases), then the call's status word:
// nonzero when a slot id would fall past the arena's n_slots (those slots are
// dropped, never written)
extern "C" int64_t carekv_store_workspace_bytes(int32_t n_jobs) { return (int64_t)n_jobs * 16 + 16; }

template <int D, int BITS>
static int launch_store(const carekv_arena& A, const carekv_store_params& sp, const uint16_t* K, const uint16_t* V,
                        const carekv_page_job* jobs, int n_jobs, const int32_t* group_ptr, int n_groups,
                        StoreWs ws, hipStream_t s) {
  const int blocks = (n_jobs + 3) / 4;
  hipLaunchKernelGGL((store_pages_kernel<D, BITS, 0>), dim3(blocks), dim3(256), 0, s, A, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(count)");
  hipLaunchKernelGGL(store_scan_kernel, dim3(n_groups), dim3(256), 0, s, A, jobs, group_ptr, ws);
  CAREKV_CHECK_LAUNCH("store_scan");
  hipLaunchKernelGGL((store_pages_kernel<D, BITS, 1>), dim3(blocks), dim3(256), 0, s, A, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(write)");
  return CAREKV_OK;
}

// The fp16 tail of a packed KIVI arena as a side-buffer arena under the
// code-page map of n_packed.
static carekv_arena kivi_tail_view(const carekv_arena& A) {
  carekv_arena At = A;
  At.base_bits = 16;
  At.scale_mode = 0;
  At.kcodes = (int8_t*)A.tail_k;
  At.vcodes = (int8_t*)A.tail_v;
  At.kivi_packed = 0;
  At.code_pages = A.tail_pages;
  At.code_page_off = A.n_packed;
  return At;
}

// Both kinds of page of a packed KIVI arena in one slot allocation: the
// count passes of the prefix and the tail, the scan over all jobs, then the
// two write passes.
template <int D>
static int launch_store_kivi(const carekv_arena& A, const carekv_store_params& sp, const uint16_t* K,
                             const uint16_t* V, const carekv_page_job* jobs, int n_jobs, const int32_t* group_ptr,
                             int n_groups, StoreWs ws, hipStream_t s) {
  const carekv_arena At = kivi_tail_view(A);
  const int blocks = (n_jobs + 3) / 4;
  hipLaunchKernelGGL((store_pages_kernel<D, 2, 0>), dim3(blocks), dim3(256), 0, s, A, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(count, packed KIVI prefix)");
  hipLaunchKernelGGL((store_pages_kernel<D, 16, 0>), dim3(blocks), dim3(256), 0, s, At, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(count, packed KIVI tail)");
  hipLaunchKernelGGL(store_scan_kernel, dim3(n_groups), dim3(256), 0, s, A, jobs, group_ptr, ws);
  CAREKV_CHECK_LAUNCH("store_scan");
  hipLaunchKernelGGL((store_pages_kernel<D, 2, 1>), dim3(blocks), dim3(256), 0, s, A, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(write, packed KIVI prefix)");
  hipLaunchKernelGGL((store_pages_kernel<D, 16, 1>), dim3(blocks), dim3(256), 0, s, At, sp, K, V, jobs, n_jobs, ws);
  CAREKV_CHECK_LAUNCH("store_pages(write, packed KIVI tail)");
  return CAREKV_OK;
}

extern "C" int carekv_store_pages(const carekv_arena* arena, const carekv_store_params* sp, const uint16_t* K,
                                  const uint16_t* V, const carekv_page_job* jobs_dev, int32_t n_jobs,
                                  const int32_t* group_ptr_dev, int32_t n_groups, void* workspace,
                                  void* stream) {
  CAREKV_REQUIRE(arena && sp && K && V && jobs_dev && group_ptr_dev && workspace, "null argument");
  CAREKV_REQUIRE(n_jobs >= 0 && n_groups >= 0, "negative sizes");
  if (n_jobs == 0) return CAREKV_OK;
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.residual_bits == 4, "kernels support residual_bits=4");
  CAREKV_REQUIRE(sp->sketch_proj != nullptr, "sketch_proj is required");
  StoreWs ws{(int32_t*)workspace};
  hipStream_t s = (hipStream_t)stream;
  if (A.kivi_packed) {
    CAREKV_REQUIRE(sp->k_hat && sp->v_hat && sp->k_codes_in && sp->v_codes_in && sp->v_scale_in,
                   "a packed KIVI arena stores from k_hat, v_hat, k_codes_in, v_codes_in and v_scale_in");
    CAREKV_REQUIRE(!sp->keep_base, "keep_base is built for the uniform packed bases");
    if (A.head_dim == 64) return launch_store_kivi<64>(A, *sp, K, V, jobs_dev, n_jobs, group_ptr_dev, n_groups, ws, s);
    return launch_store_kivi<128>(A, *sp, K, V, jobs_dev, n_jobs, group_ptr_dev, n_groups, ws, s);
  }
  if (A.base_bits == 16) {
    CAREKV_REQUIRE(sp->k_hat && sp->v_hat, "the fp16 base (base_bits=16) needs k_hat and v_hat");
    CAREKV_REQUIRE(!sp->keep_base, "keep_base (streaming store) is built for the packed bases");
    if (A.head_dim == 64) return launch_store<64, 16>(A, *sp, K, V, jobs_dev, n_jobs, group_ptr_dev, n_groups, ws, s);
    return launch_store<128, 16>(A, *sp, K, V, jobs_dev, n_jobs, group_ptr_dev, n_groups, ws, s);
  }
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    return launch_store<decltype(d)::value, decltype(b)::value>(A, *sp, K, V, jobs_dev, n_jobs, group_ptr_dev,
                                                                n_groups, ws, s);
  });
}

namespace {
int append_any(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* dest_dev,
               int32_t n_rows, const CodedRows& cr, void* stream);
}  // namespace

extern "C" int carekv_append_rows(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows,
                                  const int32_t* dest_dev, int32_t n_rows, void* stream) {
  CAREKV_REQUIRE(k_rows && v_rows, "null argument");
  return append_any(arena, k_rows, v_rows, dest_dev, n_rows, CodedRows{nullptr, nullptr, nullptr, nullptr}, stream);
}

extern "C" int carekv_append_coded_rows(const carekv_arena* arena, const int8_t* k_codes, const uint16_t* k_scale,
                                        const int8_t* v_codes, const uint16_t* v_scale, const int32_t* dest_dev,
                                        int32_t n_rows, void* stream) {
  CAREKV_REQUIRE(k_codes && k_scale && v_codes && v_scale, "null argument");
  CAREKV_REQUIRE(arena && arena->base_bits != 16, "coded rows need a packed base");
  return append_any(arena, nullptr, nullptr, dest_dev, n_rows, CodedRows{k_codes, k_scale, v_codes, v_scale}, stream);
}

namespace {
int append_any(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* dest_dev,
               int32_t n_rows, const CodedRows& cr, void* stream) {
  CAREKV_REQUIRE(arena && dest_dev, "null argument");
  if (n_rows <= 0) return CAREKV_OK;
  CAREKV_REQUIRE(check_arena(*arena), last_error_buf());
  carekv_arena A = *arena;
  if (A.kivi_packed) {  // decode rows go to the fp16 tail
    CAREKV_REQUIRE(k_rows && v_rows, "a packed KIVI arena appends fp16 rows");
    A = kivi_tail_view(*arena);
  }
  hipStream_t s = (hipStream_t)stream;
  if (A.base_bits == 16) {
    if (A.head_dim == 64)
      hipLaunchKernelGGL(append_hat_rows_kernel<64>, dim3((n_rows + 3) / 4), dim3(256), 0, s, A, k_rows, v_rows,
                         dest_dev, n_rows);
    else
      hipLaunchKernelGGL(append_hat_rows_kernel<128>, dim3((n_rows + 3) / 4), dim3(256), 0, s, A, k_rows, v_rows,
                         dest_dev, n_rows);
    CAREKV_CHECK_LAUNCH("append_hat_rows");
    return CAREKV_OK;
  }
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    hipLaunchKernelGGL((append_rows_kernel<decltype(d)::value, decltype(b)::value>), dim3((n_rows + 3) / 4),
                       dim3(256), 0, s, A, k_rows, v_rows, dest_dev, n_rows, cr);
    CAREKV_CHECK_LAUNCH("append_rows");
    return CAREKV_OK;
  });
}
}  // namespace

extern "C" int carekv_read_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                                 const int32_t* page_ids_dev, const int32_t* row_start_dev, int8_t* kc, uint16_t* ks,
                                 int8_t* vc, uint16_t* vs, void* stream) {
  CAREKV_REQUIRE(arena && row_start_dev && kc && ks && vc && vs, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(seq >= 0 && seq < A.n_seq && kv_head >= 0 && kv_head < A.n_kv_heads, "seq/kv_head out of range");
  CAREKV_REQUIRE(n_pages >= 0 && (page_ids_dev || n_pages <= A.max_pages), "n_pages out of range");
  CAREKV_REQUIRE(A.base_bits != 16 && !A.kivi_packed,
                 "the fp16 and packed KIVI bases have no uniform codes to read: use carekv_read_hat_pages");
  if (n_pages == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    hipLaunchKernelGGL((read_pages_kernel<decltype(d)::value, decltype(b)::value>), dim3(n_pages), dim3(64), 0, s,
                       A, seq, kv_head, n_pages, page_ids_dev, row_start_dev, kc, ks, vc, vs);
    CAREKV_CHECK_LAUNCH("read_pages");
    return CAREKV_OK;
  });
}

extern "C" int carekv_quantize_rows(const uint16_t* x, int32_t rows, int32_t D, int32_t bits, int32_t group,
                                    int32_t pack, int8_t* codes, uint16_t* scale, void* stream) {
  CAREKV_REQUIRE(x && codes && scale, "null argument");
  CAREKV_REQUIRE(group == 32 && D % 32 == 0 && D > 0, "kernels support group_size=32 and D % 32 == 0");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  if (rows <= 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int n = rows * (D / 32);
  const int blocks = (n + 255) / 256;
  switch (bits) {
    case 2: hipLaunchKernelGGL(quantize_rows_kernel<2>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
    case 3: hipLaunchKernelGGL(quantize_rows_kernel<3>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
    default: hipLaunchKernelGGL(quantize_rows_kernel<4>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
  }
  CAREKV_CHECK_LAUNCH("quantize_rows");
  return CAREKV_OK;
}

extern "C" int carekv_kivi_codes(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits,
                                 int32_t per_channel, int8_t* codes, uint16_t* scale, void* stream) {
  CAREKV_REQUIRE(x && codes && scale, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D <= 1024 && n_mat >= 0 && rows >= 0, "bad shape");
  if (n_mat == 0 || rows == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (per_channel) {
    CAREKV_REQUIRE(n_mat <= 65535 * 1024, "too many matrices");
    hipLaunchKernelGGL(kivi_channel_codes_kernel, dim3(n_mat, (D + 63) / 64), dim3(256), 0, s, x, rows, D, bits,
                       codes, scale);
  } else {
    const long n_rows = (long)n_mat * rows;
    CAREKV_REQUIRE((n_rows + 3) / 4 <= 0x7fffffffL, "too many rows");
    hipLaunchKernelGGL(kivi_token_codes_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, s, x, n_rows, D,
                       bits, codes, scale);
  }
  CAREKV_CHECK_LAUNCH("kivi_codes");
  return CAREKV_OK;
}

extern "C" int carekv_read_hat_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                                     const int32_t* page_ids_dev, const int32_t* row_start_dev, uint16_t* k_hat,
                                     uint16_t* v_hat, void* stream) {
  CAREKV_REQUIRE(arena && row_start_dev && k_hat && v_hat, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.base_bits == 16 || A.kivi_packed, "carekv_read_hat_pages reads the fp16 and packed KIVI bases");
  CAREKV_REQUIRE(seq >= 0 && seq < A.n_seq && kv_head >= 0 && kv_head < A.n_kv_heads, "seq/kv_head out of range");
  CAREKV_REQUIRE(n_pages >= 0 && (page_ids_dev || n_pages <= A.max_pages), "n_pages out of range");
  if (n_pages == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (A.head_dim == 64)
    hipLaunchKernelGGL(read_hat_pages_kernel<64>, dim3(n_pages), dim3(64), 0, s, A, seq, kv_head, n_pages,
                       page_ids_dev, row_start_dev, k_hat, v_hat);
  else
    hipLaunchKernelGGL(read_hat_pages_kernel<128>, dim3(n_pages), dim3(64), 0, s, A, seq, kv_head, n_pages,
                       page_ids_dev, row_start_dev, k_hat, v_hat);
  CAREKV_CHECK_LAUNCH("read_hat_pages");
  return CAREKV_OK;
}

extern "C" int carekv_kivi_qdq(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits,
                               int32_t per_channel, uint16_t* out, void* stream) {
  CAREKV_REQUIRE(x && out, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D <= 1024 && n_mat >= 0 && rows >= 0, "bad shape");
  if (n_mat == 0 || rows == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (per_channel) {
    CAREKV_REQUIRE(n_mat <= 65535 * 1024, "too many matrices");
    hipLaunchKernelGGL(kivi_channel_kernel, dim3(n_mat, (D + 63) / 64), dim3(256), 0, s, x, rows, D, bits, out);
  } else {
    const long n_rows = (long)n_mat * rows;
    CAREKV_REQUIRE((n_rows + 3) / 4 <= 0x7fffffffL, "too many rows");
    hipLaunchKernelGGL(kivi_token_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, s, x, n_rows, D, bits, out);
  }
  CAREKV_CHECK_LAUNCH("kivi_qdq");
  return CAREKV_OK;
}
