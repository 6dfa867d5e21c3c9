// Select pass of the CARE-KV decode: one work-group per (query head of the
// GQA group, kv head, sequence), after the streaming kernel.
//   * combines the split partials into the softmax statistics (M, L) and
//     O_base of the query (attention.py:1015-1022);
//   * scores every stored slot from the page records: the query-aware K
//     score ||dS * A(1-A)|| * ||V_page|| * sens (attention.py:167-184, 704-760)
//     and the V score mass * v_err * sens (attention.py:780-790, with
//     v_err already scaled by sens in build_v_slot_index);
//   * normalises each kind by its mean score (attention.py:830-844),
//     resolves the read budgets (residual_router.py:37-76) and selects the
//     joint or per-kind top-k with ties toward the lowest candidate index
//     (attention.py:856-875), by a 4-pass radix select on the float bits;
//   * writes the per-page selection masks for the apply kernel, the
//     optional diag list, and with correction off the output itself.
// Candidate index: K slot r of page p -> p*k_cap + r; V block r of page p
// -> np*k_cap + p*v_cap + r (the reference's [score_K | score_V] order).
#include <limits.h>

#include "block_util.h"
#include "decode_common.h"
#include "host_util.h"

namespace carekv {

constexpr float kEps = 1e-6f;  // residual_router.py:34

// Slot ids outside the arena read as "no slot" (as in the streaming kernel).
__device__ __forceinline__ bool slot_ok(const carekv_arena& A, int s) { return s >= 0 && s < A.n_slots; }

struct CandView {
  const float* sc;
  int nK, nV;
  int norm;
  float divK, divV, lamK, lamV;
};

// Non-negative float bits of candidate i, or -1 for an empty position.
__device__ __forceinline__ int cand_bits(const CandView& cv, int i) {
  float x = cv.sc[i];
  if (!(x >= 0.f)) return -1;
  if (cv.norm) x = i < cv.nK ? (x / cv.divK) * cv.lamK : (x / cv.divV) * cv.lamV;
  return (int)(__float_as_uint(x) & 0x7fffffffu);
}

struct Sel {
  uint32_t tau;  // threshold bits
  int take;      // candidates equal to tau to take (lowest index first)
  int eq;        // candidates equal to tau
  bool on;
};

// k-th largest of the candidates [lo, hi).
__device__ Sel radix_select(const CandView& cv, int lo, int hi, int k, int* hist, BlockScratch& bs) {
  Sel r{0u, INT_MAX, 0, true};
  int cnt = 0;
  for (int i = lo + threadIdx.x; i < hi; i += kBlock) cnt += cand_bits(cv, i) >= 0;
  const int nvalid = block_isum(cnt, bs);
  if (nvalid <= k) return r;  // every valid candidate is taken
  uint32_t prefix = 0, mask = 0;
  int krem = k;
  const int lane = threadIdx.x & 63;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int i = lo + threadIdx.x; i < hi; i += kBlock) {
      const int u = cand_bits(cv, i);
      if (u >= 0 && ((uint32_t)u & mask) == prefix) atomicAdd(&hist[((uint32_t)u >> shift) & 255u], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l covers digits 255-4l .. 252-4l (descending)
      int c[4], loc = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) { c[i] = hist[255 - 4 * lane - i]; loc += c[i]; }
      int incl = loc;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      const int excl = incl - loc;
      if (excl < krem && krem <= incl) {  // exactly one lane
        int cum = excl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (cum + c[i] >= krem) {
            bs.bc[0] = 255 - 4 * lane - i;
            bs.bc[1] = krem - cum;
            bs.bc[2] = c[i];
            break;
          }
          cum += c[i];
        }
      }
    }
    __syncthreads();
    prefix |= (uint32_t)bs.bc[0] << shift;
    krem = bs.bc[1];
    mask |= 255u << shift;
    r.eq = bs.bc[2];
    __syncthreads();
  }
  r.tau = prefix;
  r.take = krem;
  return r;
}

template <int D>
__global__ __launch_bounds__(256) void decode_select_kernel(carekv_arena A, DecodeArgs a) {
  constexpr int NCG = D / 32;
  __shared__ BlockScratch bs;
  __shared__ int hist[256];
  const int qq = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const int seq_raw = a.seq_slot[b], np_raw = a.n_pages[b];
  const bool row_ok = seq_raw >= 0 && seq_raw < A.n_seq && np_raw >= 0 && np_raw <= a.Pmax;
  const int np = row_ok ? np_raw : 0;
  const int seq = row_ok ? seq_raw : 0;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const int tid = threadIdx.x;
  const long bq = (long)bk * GQ + qq;
  uint16_t* outp = a.out + ((long)b * a.Hq + kvh * GQ + qq) * D;
  int32_t* diagp = a.diag ? a.diag + ((long)b * a.Hq + kvh * GQ + qq) * a.diag_cap : nullptr;

  // ---- softmax statistics and O_base from the split partials
  float mloc = -INFINITY;
  for (int s = tid; s < a.nsplit; s += kBlock) mloc = fmaxf(mloc, a.pml[(((long)bk * a.nsplit + s) * 16 + qq) * 2]);
  const float M = block_max(mloc, bs);
  float lloc = 0.f;
  if (M != -INFINITY)
    for (int s = tid; s < a.nsplit; s += kBlock) {
      const long base = ((long)bk * a.nsplit + s) * 16 + qq;
      const float ms = a.pml[base * 2];
      if (ms != -INFINITY) lloc += a.pml[base * 2 + 1] * __builtin_amdgcn_exp2f(ms - M);
    }
  const float L = block_sum(lloc, bs);
  for (int d = tid; d < D; d += kBlock) {
    float O = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < a.nsplit; ++s) {
        const long base = ((long)bk * a.nsplit + s) * 16 + qq;
        const float ms = a.pml[base * 2];
        if (ms != -INFINITY) O += a.po[base * D + d] * __builtin_amdgcn_exp2f(ms - M);
      }
    const float ob = L > 0.f ? O / L : 0.f;
    if (a.correction) a.ob[bq * D + d] = ob;
    else outp[d] = f2h(ob);
  }
  if (tid == 0) { a.ml[bq * 2] = M; a.ml[bq * 2 + 1] = L; }
  if (!a.correction) {
    if (diagp)
      for (int i = tid; i < a.diag_cap; i += kBlock) diagp[i] = -1;
    return;
  }

  // ---- score every stored slot
  const int k_cap = a.k_cap, v_cap = a.v_cap;
  const int nK = np * k_cap, nV = np * v_cap;
  const float* recq = a.rec + bq * a.Pmax * a.F;
  float* sc = a.scores + bq * a.ncand;
  uint8_t* maskq = a.mask + bq * a.Pmax;
  float sumK = 0.f, sumV = 0.f;
  int cntK = 0, cntV = 0;
  const bool have_stats = L > 0.f;
  for (int p = tid; p < np; p += kBlock) {
    const long pg = pg_base + p;
    const int nv = A.valid[pg];
    const bool ok = have_stats && nv > 0 && A.has_meta[pg];
    const float* r = recq + (long)p * a.F;
    const float c = ok ? __builtin_amdgcn_exp2f(r[0] - M) / L : 0.f;
    const float vnorm = ok ? sqrtf(A.v_sq[pg]) : 0.f;
    int rk = 0;
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      if (!ok || !slot_ok(A, A.k_slot[pg * NCG + cg]) || rk >= k_cap) continue;
      const float M2 = r[1 + 3 * rk], M3 = r[2 + 3 * rk], M4 = r[3 + 3 * rk];
      const float q2 = c * c * (M2 - c * (2.f * M3 - c * M4));
      float ks = sqrtf(fmaxf(q2, 0.f)) * vnorm;
      if (!isfinite(ks)) ks = 0.f;
      ks = ks * a.sens;
      sc[p * k_cap + rk] = ks;
      sumK += ks;
      ++cntK;
      ++rk;
    }
    for (; rk < k_cap; ++rk) sc[p * k_cap + rk] = -1.f;
    int rv = 0;
#pragma unroll
    for (int vb = 0; vb < kVtb; ++vb) {
      if (!ok || !slot_ok(A, A.v_slot[pg * kVtb + vb]) || rv >= v_cap) continue;
      float vsc = -1.f;
      if (vb * kVtb < nv) {
        const float verr_s = (float)((double)h2f(A.v_err[pg * kVtb + vb]) * a.sens_d);
        vsc = (c * r[1 + 3 * k_cap + rv]) * verr_s;
        vsc = vsc * a.sens;
        sumV += vsc;
        ++cntV;
      }
      sc[nK + p * v_cap + rv] = vsc;
      ++rv;
    }
    for (; rv < v_cap; ++rv) sc[nK + p * v_cap + rv] = -1.f;
  }
  const float tK = block_sum(sumK, bs), tV = block_sum(sumV, bs);
  const int n_k = block_isum(cntK, bs), n_v = block_isum(cntV, bs);

  // ---- read budgets (residual_router.py:37-76 via attention.py:662-670)
  const bool want_k = (a.kind == 0 || a.kind == 1) && n_k > 0;
  const bool want_v = (a.kind == 0 || a.kind == 2) && n_v > 0;
  const int totk = want_k ? n_k : 0, totv = want_v ? n_v : 0;
  int bud_k, bud_v;
  if (!a.budget_ratio) {
    bud_k = a.abs_k; bud_v = a.abs_v;
  } else {
    bud_k = (a.ratio_k > 0.0 && totk > 0) ? max(1, (int)((double)totk * a.ratio_k)) : 0;
    bud_v = (a.ratio_v > 0.0 && totv > 0) ? max(1, (int)((double)totv * a.ratio_v)) : 0;
  }
  if (a.kind == 2) bud_k = 0;
  if (a.kind == 1) bud_v = 0;
  bud_k = min(bud_k, totk);
  bud_v = min(bud_v, totv);
  const bool haveK = want_k && bud_k > 0, haveV = want_v && bud_v > 0;
  const bool do_norm = a.normalize && a.kind == 0 && haveK && haveV;
  const bool joint = a.joint && a.kind == 0 && haveK && haveV;
  const CandView cv{sc, nK, nV, do_norm ? 1 : 0,
                    n_k > 0 ? fmaxf(tK / (float)n_k, kEps) : kEps,
                    n_v > 0 ? fmaxf(tV / (float)n_v, kEps) : kEps, a.lam_k, a.lam_v};

  // ---- thresholds
  Sel sk{0u, 0, 0, false}, sv{0u, 0, 0, false};
  if (joint) {
    const int mb = min(bud_k + bud_v, n_k + n_v);
    sk = radix_select(cv, 0, nK + nV, mb, hist, bs);
    sv = sk;
  } else {
    if (haveK) sk = radix_select(cv, 0, nK, min(bud_k, n_k), hist, bs);
    if (haveV) sv = radix_select(cv, nK, nK + nV, min(bud_v, n_v), hist, bs);
  }

  // ---- masks and diag: a sweep over the K candidates, then the V ones
  int sel_run = 0, eqK_seen = 0;
  for (int kind = 0; kind < 2; ++kind) {
    const Sel& s = kind == 0 ? sk : sv;
    const int cap = kind == 0 ? k_cap : v_cap;
    const int seg0 = kind == 0 ? 0 : nK;
    const bool need_rank = s.on && s.take < s.eq;
    int eq_run = (kind == 1 && joint) ? eqK_seen : 0;
    for (int p0 = 0; p0 < np; p0 += kBlock) {
      const int p = p0 + tid;
      const bool pv = p < np;
      int u[4] = {-1, -1, -1, -1};
      int eqc = 0;
      if (pv && s.on)
        for (int r = 0; r < cap; ++r) {
          u[r] = cand_bits(cv, seg0 + p * cap + r);
          eqc += u[r] >= 0 && (uint32_t)u[r] == s.tau;
        }
      int eq_before = 0;
      if (need_rank) {
        int tot;
        eq_before = block_excl_scan(eqc, bs, &tot) + eq_run;
        eq_run += tot;
      }
      unsigned bits = 0;
      for (int r = 0; r < cap; ++r) {
        if (u[r] < 0) continue;
        const uint32_t x = (uint32_t)u[r];
        bool take = x > s.tau;
        if (x == s.tau) { take = eq_before < s.take; ++eq_before; }
        if (take) bits |= 1u << r;
      }
      if (pv) {
        if (kind == 0) maskq[p] = (uint8_t)bits;
        else maskq[p] = (uint8_t)(maskq[p] | (bits << 4));
      }
      if (diagp) {
        int tot;
        int pos = block_excl_scan(__popc(bits), bs, &tot) + sel_run;
        sel_run += tot;
        if (bits) {
          const long pg = pg_base + p;
          int rr = 0;
          const int nsub = kind == 0 ? NCG : kVtb;
          for (int sub = 0; sub < nsub && rr < cap; ++sub) {
            const int slot = kind == 0 ? A.k_slot[pg * NCG + sub] : A.v_slot[pg * kVtb + sub];
            if (!slot_ok(A, slot)) continue;
            if ((bits >> rr) & 1u) {
              if (pos < a.diag_cap) diagp[pos] = (kind << 30) | (p << 3) | sub;
              ++pos;
            }
            ++rr;
          }
        }
      }
    }
    if (kind == 0) eqK_seen = eq_run;  // K ties rank before the V ones of a joint selection
  }
  if (diagp)
    for (int i = sel_run + tid; i < a.diag_cap; i += kBlock) diagp[i] = -1;
}

int launch_decode_select(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.GQ, A.n_kv_heads, a.B);
  if (A.head_dim == 64) {
    hipLaunchKernelGGL(decode_select_kernel<64>, grid, dim3(kBlock), 0, s, A, a);
  } else if (A.head_dim == 128) {
    hipLaunchKernelGGL(decode_select_kernel<128>, grid, dim3(kBlock), 0, s, A, a);
  } else {
    set_error("unsupported head_dim %d", A.head_dim);
    return CAREKV_EINVAL;
  }
  CAREKV_CHECK_LAUNCH("decode_select");
  return CAREKV_OK;
}

}  // namespace carekv
