// Select pass of the CARE-KV decode: one work-group per (query head of the
// GQA group, kv head, sequence), after the streaming kernel.
//   * combines the split partials into the softmax statistics (M, L) of the
//     query (with correction off, also O_base, which is then the output:
//     attention.py:1015-1022);
//   * scores every stored slot from the page records: the query-aware K
//     score ||dS * A(1-A)|| * ||V_page|| * sens (attention.py:167-184, 704-760)
//     or, with the sketch proxy, mass * |q_cg P . k_sketch| * boundary *
//     vdiff * sens (attention.py:718-725) from the decode_proxy_kernel
//     records, and the V score mass * v_err * sens (attention.py:780-790,
//     with v_err already scaled by sens in build_v_slot_index);
//   * normalises each kind by its mean score (attention.py:830-844),
//     resolves the read budgets (residual_router.py:37-76) and selects the
//     joint or per-kind top-k with ties toward the lowest candidate index
//     (attention.py:856-875), by a radix select on the float bits;
//   * writes the per-page selection masks for the apply kernel and the
//     optional diag list.
// Candidate index: K slot r of page p -> p*k_cap + r; V block r of page p
// -> np*k_cap + p*v_cap + r (the reference's [score_K | score_V] order).
#include <limits.h>

#include <type_traits>

#include "block_util.h"
#include "decode_common.h"
#include "host_util.h"

namespace carekv {

constexpr float kEps = 1e-6f;  // residual_router.py:34

// v_sqrt_f32 and v_exp_f32 read and give fp32 denormals as zero, while the
// reference's fp32 arithmetic keeps them: the attention mass and the K
// score terms of a page far below the maximum fall under 2^-126 there and
// still rank candidates.  These scale such arguments into the normal range.
__device__ __forceinline__ float sqrt_dn(float x) {
  return x < 0x1p-100f ? __builtin_amdgcn_sqrtf(x * 0x1p100f) * 0x1p-50f : __builtin_amdgcn_sqrtf(x);
}
__device__ __forceinline__ float exp2_dn(float x) {
  return x < -126.f ? __builtin_amdgcn_exp2f(x + 64.f) * 0x1p-64f : __builtin_amdgcn_exp2f(x);
}
// The reference sums the per-token squares (dS_t A_t (1 - A_t))^2 in fp32;
// when even sum_t (dS_t A_t)^2 = c^2 (M2 + D* e*^2) is at most 2^-150,
// every one of them rounds to zero there and its K score is exactly 0.
__device__ __forceinline__ bool kscore_underflows(float c, float M2, float Ds, float es) {
  return c * sqrt_dn(M2 + Ds * (es * es)) <= 0x1p-75f;
}

template <int N>
__device__ __forceinline__ void load_slots(int* out, const int32_t* p) {
  if constexpr (N == 4) {
    const int4 v = *reinterpret_cast<const int4*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    static_assert(N == 2, "slot row");
    const int2 v = *reinterpret_cast<const int2*>(p);
    out[0] = v.x; out[1] = v.y;
  }
}

// Slot ids outside the arena read as "no slot" (as in the streaming kernel).
__device__ __forceinline__ bool slot_ok(const carekv_arena& A, int s) { return s >= 0 && s < A.n_slots; }

struct Sel {
  uint32_t tau;  // threshold key
  int take;      // candidates equal to tau to take (lowest index first)
  int eq;        // candidates equal to tau
  bool on;
};

// k-th largest key of the candidates [lo, hi) (key -1: empty position),
// by 8-bit radix passes from the top; two histograms (one per wave pair)
// spread the LDS atomics.
__device__ __forceinline__ Sel radix_select(const int* key, int lo, int hi, int k, int (*hist)[256], BlockScratch& bs) {
  Sel r{0u, INT_MAX, 0, true};
  int cnt = 0;
  for (int i = lo + threadIdx.x; i < hi; i += kBlock) cnt += key[i] >= 0;
  const int nvalid = block_isum_fast(cnt, bs);
  if (nvalid <= k) return r;  // every valid candidate is taken
  uint32_t prefix = 0, mask = 0;
  int krem = k;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
#pragma unroll
    for (int c = 0; c < 2; ++c) hist[c][threadIdx.x] = 0;
    __syncthreads();
    for (int i = lo + threadIdx.x; i < hi; i += kBlock) {
      const int u = key[i];
      if (u >= 0 && ((uint32_t)u & mask) == prefix) atomicAdd(&hist[w >> 1][((uint32_t)u >> shift) & 255u], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l covers digits 255-4l .. 252-4l (descending)
      int c[4], loc = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 255 - 4 * lane - i;
        c[i] = hist[0][d] + hist[1][d];
        loc += c[i];
      }
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
    const int in_bin = bs.bc[2];
    __syncthreads();
    if (krem == in_bin) {  // the whole bin is taken: every key >= prefix is selected
      r.tau = prefix; r.take = INT_MAX; r.eq = 0;
      return r;
    }
    r.eq = in_bin;
  }
  r.tau = prefix;
  r.take = krem;
  return r;
}

// Selection masks of one query from the thresholds: keys above tau are
// taken, ties at tau in candidate order (V ties of a joint selection after
// every K tie).  which: bit 0 rewrites the K bits of the mask bytes, bit 1
// the V bits; the other kind's bits are kept.  Each thread owns pages
// tid, tid + kBlock, ...
__device__ __forceinline__ void write_masks(const int* key, uint8_t* maskq, int np, int k_cap, int v_cap, int nK, const Sel& sk,
                            const Sel& sv, bool joint, int which, BlockScratch& bs) {
  const int tid = threadIdx.x;
  const bool rankK = sk.on && sk.take < sk.eq, rankV = sv.on && sv.take < sv.eq;
  int eqK_total = 0;
  if (joint && rankK) {  // V ties of a joint selection rank after every K tie
    int c = 0;
    for (int i = tid; i < nK; i += kBlock) c += key[i] >= 0 && (uint32_t)key[i] == sk.tau;
    eqK_total = block_isum_fast(c, bs);
  }
  int eq_runK = 0, eq_runV = joint ? eqK_total : 0;
  for (int p0 = 0; p0 < np; p0 += kBlock) {
    const int p = p0 + tid;
    const bool pv = p < np;
    int uk[4] = {-1, -1, -1, -1}, uv[4] = {-1, -1, -1, -1};
    int eqk = 0, eqv = 0;
    if (pv) {
      if (sk.on)
        for (int r = 0; r < k_cap; ++r) {
          uk[r] = key[p * k_cap + r];
          eqk += uk[r] >= 0 && (uint32_t)uk[r] == sk.tau;
        }
      if (sv.on)
        for (int r = 0; r < v_cap; ++r) {
          uv[r] = key[nK + p * v_cap + r];
          eqv += uv[r] >= 0 && (uint32_t)uv[r] == sv.tau;
        }
    }
    int ek = 0, ev = 0;
    if (rankK) { int tot; ek = block_excl_scan(eqk, bs, &tot) + eq_runK; eq_runK += tot; }
    if (rankV) { int tot; ev = block_excl_scan(eqv, bs, &tot) + eq_runV; eq_runV += tot; }
    unsigned bits = 0;
    for (int r = 0; r < k_cap; ++r) {
      if (uk[r] < 0) continue;
      const uint32_t x = (uint32_t)uk[r];
      bool take = x > sk.tau;
      if (x == sk.tau) { take = ek < sk.take; ++ek; }
      if (take) bits |= 1u << r;
    }
    for (int r = 0; r < v_cap; ++r) {
      if (uv[r] < 0) continue;
      const uint32_t x = (uint32_t)uv[r];
      bool take = x > sv.tau;
      if (x == sv.tau) { take = ev < sv.take; ++ev; }
      if (take) bits |= 1u << (4 + r);
    }
    if (pv) {
      const unsigned keep = (which & 1 ? 0u : 15u) | (which & 2 ? 0u : 0xf0u);
      maskq[p] = (uint8_t)((maskq[p] & keep) | bits);
    }
  }
}

constexpr int kLdsCand = 8192;  // candidates kept in LDS (32 KB); more go to the workspace

// Work-groups are dealt to the 8 XCDs round-robin by linear id; the GQ
// query work-groups of one (sequence, kv head) share its page tables, so
// they are mapped to one XCD (one L2): within a window of 8*GQ ids, XCD x
// gets pair window*8 + x for queries 0..GQ-1.
constexpr int kXcd = 8;

// PX: K scores from the sketch proxy records instead of the moments.
// K1: k_cap = v_cap = 1 (records [m_ref, M2, M3, M4, D*, e*, mass]), the common
// store budget of one K and one V slot per page, scored without the
// generic rank loops.
// LC: the candidates' scores and keys live in LDS (ncand <= kLdsCand), else
// in the workspace; a compile-time choice, so that every access has a known
// address space (a generic pointer makes each one a flat access, and the
// waits around flat accesses cover every outstanding load)
template <int D, bool PX, bool K1, bool LC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8))) void decode_select_kernel(carekv_arena A, DecodeArgs a) {
  constexpr int NCG = D / 32;
  constexpr int FMAX = 2 + 4 * NCG + kVtb;
  __shared__ BlockScratch bs;
  __shared__ int hist[2][256];  // one histogram per wave pair
  __shared__ float s_qs[NCG * 64];  // q_cg P per channel group (sketch proxy)
  extern __shared__ float s_cand[];  // ncand floats when they fit (size set at launch)
  const int GQ = a.GQ;
  // prefill rows: the latest (longest) rows first (a window keeps its XCD)
  const int win_d = blockIdx.x / (kXcd * GQ), rem = blockIdx.x % (kXcd * GQ);
  const int win = a.pf ? (int)(gridDim.x / (kXcd * GQ)) - 1 - win_d : win_d;
  const int pair = win * kXcd + rem % kXcd, qq = rem / kXcd;
  if (pair >= a.B * A.n_kv_heads) return;
  const int kvh = pair % A.n_kv_heads, b = pair / A.n_kv_heads;
  const int bk = b * A.n_kv_heads + kvh;
  const EntryRow er = entry_row(A, a, b);
  const int np = er.np, seq = er.seq;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const int tid = threadIdx.x;
  const long bq = (long)bk * GQ + qq;
  int32_t* diagp = nullptr;
  if (a.diag) {
    if (a.pf) {  // prefill rows: the column's (row, head); padding columns write nothing
      const PfCol x = pf_col(a, b, kvh, qq);
      diagp = x.ok ? a.diag + pf_row_off(a, x) * a.diag_cap : nullptr;
    } else {
      diagp = a.diag + ((long)b * a.Hq + kvh * GQ + qq) * a.diag_cap;
    }
  }

  // ---- softmax statistics from the split partials
  const int nsr = splits_read(a, b);
  float mloc = -INFINITY;
  for (int s = tid; s < nsr; s += kBlock) mloc = fmaxf(mloc, a.pml[(((long)bk * a.nsplit + s) * 16 + qq) * 2]);
  const float M = block_max_fast(mloc, bs);
  float lloc = 0.f;
  if (M != -INFINITY)
    for (int s = tid; s < nsr; s += kBlock) {
      const long base = ((long)bk * a.nsplit + s) * 16 + qq;
      const float ms = a.pml[base * 2];
      if (ms != -INFINITY) lloc += a.pml[base * 2 + 1] * __builtin_amdgcn_exp2f(ms - M);
    }
  const float L = block_sum_fast(lloc, bs);
  if (tid == 0) { a.ml[bq * 2] = M; a.ml[bq * 2 + 1] = L; }
  if (!a.correction) {
    // base attention only: O_base is the output
    uint16_t* outp = a.out + ((long)b * a.Hq + kvh * GQ + qq) * D;
    for (int d = tid; d < D; d += kBlock) {
      float O = 0.f;
      if (M != -INFINITY)
#pragma unroll 8
        for (int s = 0; s < nsr; ++s) {
          const long base = ((long)bk * a.nsplit + s) * 16 + qq;
          const float ms = a.pml[base * 2];
          if (ms != -INFINITY) O += a.po[base * D + d] * __builtin_amdgcn_exp2f(ms - M);
        }
      outp[d] = f2h(L > 0.f ? O / L : 0.f);
    }
    if (diagp)
      for (int i = tid; i < a.diag_cap; i += kBlock) diagp[i] = -1;
    return;
  }

  // ---- q sketches q_cg P (fp32, attention.py:722) for the proxy
  const int skd = A.sketch_dim;
  if constexpr (PX) {
    const uint16_t* qg = a.q + ((long)b * a.Hq + kvh * GQ + qq) * D;
    if (a.pf) {  // prefill rows: the column's (row, head); a padding column sketches zero
      const PfCol x = pf_col(a, b, kvh, qq);
      qg = x.ok ? a.q + pf_row_off(a, x) * D : nullptr;
    }
    for (int i = tid; i < NCG * skd; i += kBlock) {
      const int cg = i / skd, j = i % skd;
      float acc = 0.f;
      if (qg)
        for (int c = 0; c < 32; ++c) acc = fmaf(h2f(qg[cg * 32 + c]), a.sketch_proj[c * skd + j], acc);
      s_qs[cg * 64 + j] = acc;
    }
    __syncthreads();
  }

  // ---- score every stored slot (all loads of a page issued up front)
  const int k_cap = a.k_cap, v_cap = a.v_cap, F = a.F;
  const int nK = np * k_cap, nV = np * v_cap;
  const float* recq = a.rec + bq * a.Pmax * F;
  float* sc = LC ? s_cand : a.scores + bq * a.ncand;
  int* key = reinterpret_cast<int*>(sc);
  uint8_t* maskq = a.mask + bq * a.Pmax;
  // prefill rows: e_t are already the reference's attention weights
  const float invL = L > 0.f ? (a.pf ? 1.f : 1.f / L) : 0.f;
  const float* vsq_row = a.pf ? a.pf_vsq + (long)kvh * a.pf_pages : nullptr;
  float sumK = 0.f, sumV = 0.f;
  int cntK = 0, cntV = 0;
  // a page holding more stored slots than the records have room for (k_cap,
  // v_cap) cannot be scored in full: flag the call (the stored slots past
  // the caps are left out)
  bool ovf = false;
  if constexpr (PX) {  // K scores of the sketch proxy, one page per thread
#pragma unroll 1
    for (int p = tid; p < np; p += kBlock) {
      const long pg = pg_base + p;
      const bool ok = L > 0.f && A.valid[pg] > 0 && A.has_meta[pg];
      float4 px = make_float4(0.f, 0.f, 0.f, 0.f);  // mass, boundary, vdiff
      if (ok) px = *reinterpret_cast<const float4*>(a.prox + (bq * a.Pmax + p) * 4);
      int rk = 0;
#pragma unroll 1
      for (int cg = 0; cg < NCG; ++cg) {
        if (!ok || !slot_ok(A, A.k_slot[pg * NCG + cg])) continue;
        if (rk >= k_cap) { ovf = true; continue; }
        const uint16_t* ks = A.k_sketch + (pg * NCG + cg) * skd;
        float dot = 0.f;
        for (int j = 0; j < skd; ++j) dot = fmaf(s_qs[cg * 64 + j], h2f(ks[j]), dot);
        const float kp = (((px.x * fabsf(dot)) * px.y) * px.z) * a.sens;
        sc[p * k_cap + rk] = kp;
        sumK += kp;
        ++cntK;
        ++rk;
      }
      for (; rk < k_cap; ++rk) sc[p * k_cap + rk] = -1.f;
    }
  }
  if constexpr (K1 && !PX) {
    // one K and one V candidate per page: the first stored channel group
    // and the first stored V block (attention.py:540-573, 386-441 with one
    // slot per kind), scored as in the generic loop below
    const bool sens1 = a.sens_d == 1.0;
    // not unrolled: at the 64-VGPR bound of eight waves per SIMD a second
    // page in flight spills to scratch
#pragma unroll 1
    for (int p = tid; p < np; p += kBlock) {
      const long pg = pg_base + p;
      const int nv = A.valid[pg];
      const int hm = A.has_meta[pg];
      const float vsq = vsq_row ? vsq_row[p] : A.v_sq[pg];
      int ksl[NCG], vsl[kVtb];
      load_slots<NCG>(ksl, A.k_slot + pg * NCG);
      load_slots<kVtb>(vsl, A.v_slot + pg * kVtb);
      const uint2 e2 = *reinterpret_cast<const uint2*>(A.v_err + pg * kVtb);
      const float* rp = recq + (long)p * 7;
      const float r0 = rp[0], M2 = rp[1], M3 = rp[2], M4 = rp[3], Ds = rp[4], es = rp[5], E = rp[6];
      // v_sq is used only under the K-score branch; held here, so that its
      // load stays with the page's other loads instead of sinking into the
      // branch behind a wait of its own
      float vsq_h = vsq;
      asm volatile("" : "+v"(vsq_h));
      const bool ok = L > 0.f && nv > 0 && hm;
      // a select on the exponent (exp2_dn(-inf) = 0), so that the record's
      // load is issued with the page's other loads rather than behind ok
      const float c = exp2_dn(ok ? r0 - M : -INFINITY) * invL;
      int nks = 0, nvs = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) nks += slot_ok(A, ksl[cg]) ? 1 : 0;
#pragma unroll
      for (int vb = 0; vb < kVtb; ++vb) nvs += slot_ok(A, vsl[vb]) ? 1 : 0;
      ovf |= hm && (nks > 1 || nvs > 1);
      const bool kh = nks > 0;
      float ks = -1.f;
      if (ok && kh) {
        // sum_t dS^2 a^2 (1 - a)^2 = c^2 [M2 - c (2 M3 - c M4) + D* (e* (1 - a*))^2]: the page's
        // token t* evaluated directly, and c kept outside the root (c^2 of a far page underflows)
        const float wr = es * (1.f - c * es);
        const float q2 = (M2 - c * (2.f * M3 - c * M4)) + Ds * (wr * wr);
        ks = kscore_underflows(c, M2, Ds, es) ? 0.f : (c * sqrt_dn(fmaxf(q2, 0.f))) * __builtin_amdgcn_sqrtf(vsq_h);
        if (!isfinite(ks)) ks = 0.f;
        ks = ks * a.sens;
        sumK += ks;
        ++cntK;
      }
      sc[p] = ks;
      int vb1 = -1;
#pragma unroll
      for (int vb = kVtb - 1; vb >= 0; --vb)
        if (slot_ok(A, vsl[vb])) vb1 = vb;
      float vsc = -1.f;
      if (ok && vb1 >= 0 && vb1 * kVtb < nv) {
        const uint32_t ew = vb1 < 2 ? e2.x : e2.y;
        const float ve = h2f((uint16_t)(ew >> (16 * (vb1 & 1))));
        const float verr_s = sens1 ? ve : (float)((double)ve * a.sens_d);
        vsc = (c * E) * verr_s;
        vsc = vsc * a.sens;
        sumV += vsc;
        ++cntV;
      }
      sc[nK + p] = vsc;
    }
  }
#pragma unroll 1
  for (int p = tid; p < (K1 && !PX ? 0 : np); p += kBlock) {
    const long pg = pg_base + p;
    const int nv = A.valid[pg];
    const int hm = A.has_meta[pg];
    const float vsq = vsq_row ? vsq_row[p] : A.v_sq[pg];
    int ksl[NCG], vsl[kVtb];
    load_slots<NCG>(ksl, A.k_slot + pg * NCG);
    load_slots<kVtb>(vsl, A.v_slot + pg * kVtb);
    const uint2 e2 = *reinterpret_cast<const uint2*>(A.v_err + pg * kVtb);
    const uint16_t verr[kVtb] = {(uint16_t)e2.x, (uint16_t)(e2.x >> 16), (uint16_t)e2.y, (uint16_t)(e2.y >> 16)};
    float r[FMAX];
    const float* rp = recq + (long)p * F;
#pragma unroll
    for (int f = 0; f < FMAX; ++f) r[f] = f < F ? rp[f] : 0.f;
    const bool ok = L > 0.f && nv > 0 && hm;
    const float c = exp2_dn(ok ? r[0] - M : -INFINITY) * invL;
    const float vnorm = __builtin_amdgcn_sqrtf(vsq);
    if constexpr (!PX) {
      float es = 0.f;  // e of the page's token t*
#pragma unroll
      for (int f = 1; f < FMAX; ++f)
        if (f == 1 + 4 * k_cap) es = r[f];
      const float wr = es * (1.f - c * es);
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        if (!ok || !slot_ok(A, ksl[cg])) continue;
        if (rk >= k_cap) { ovf = true; continue; }
        float M2 = 0.f, M3 = 0.f, M4 = 0.f, Ds = 0.f;
#pragma unroll
        for (int j = 0; j < NCG; ++j)
          if (j == rk) { M2 = r[1 + 4 * j]; M3 = r[2 + 4 * j]; M4 = r[3 + 4 * j]; Ds = r[4 + 4 * j]; }
        const float q2 = (M2 - c * (2.f * M3 - c * M4)) + Ds * (wr * wr);
        float ks = kscore_underflows(c, M2, Ds, es) ? 0.f : (c * sqrt_dn(fmaxf(q2, 0.f))) * vnorm;
        if (!isfinite(ks)) ks = 0.f;
        ks = ks * a.sens;
        sc[p * k_cap + rk] = ks;
        sumK += ks;
        ++cntK;
        ++rk;
      }
      for (; rk < k_cap; ++rk) sc[p * k_cap + rk] = -1.f;
    }
    int rv = 0;
#pragma unroll
    for (int vb = 0; vb < kVtb; ++vb) {
      if (!ok || !slot_ok(A, vsl[vb])) continue;
      if (rv >= v_cap) { ovf = true; continue; }
      float vsc = -1.f;
      if (vb * kVtb < nv) {
        float E = 0.f;
        const int fe = 2 + 4 * k_cap + rv;
#pragma unroll
        for (int f = 1; f < FMAX; ++f)
          if (f == fe) E = r[f];
        const float verr_s = (float)((double)h2f(verr[vb]) * a.sens_d);
        vsc = (c * E) * verr_s;
        vsc = vsc * a.sens;
        sumV += vsc;
        ++cntV;
      }
      sc[nK + p * v_cap + rv] = vsc;
      ++rv;
    }
    for (; rv < v_cap; ++rv) sc[nK + p * v_cap + rv] = -1.f;
  }
  if (a.pf && tid == 0) {
    // prefill rows: the candidates of the prompt's later pages score 0
    // (A = 0 past the row) but count, as in the reference's candidate set
    // over all pages of the kv head (layer.py:514-517): their suffix counts
    const int* suf = a.pf_suf + (long)kvh * 3 * (a.pf_pages + 1);
    cntK += suf[np];
    cntV += suf[(a.pf_pages + 1) + np];
    ovf |= suf[2 * (a.pf_pages + 1) + np] != 0;
  }
  if (ovf) *a.err_flag = 1;
  float tK = sumK, tV = sumV;
  int n_k = cntK, n_v = cntV;
  block_sum4(tK, tV, n_k, n_v, bs);  // also orders the score stores before their reads

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
  // policies 2/3 and the score thresholds exist only in ResidualRouter.route,
  // which normalises each kind whenever kind is "both" (residual_router.py:292-303)
  const int pol = a.policy;
  const bool route = pol >= 2 || a.adaptive_score;
  const bool do_norm = a.normalize && a.kind == 0 && (route || (haveK && haveV));
  const bool joint = pol == 1 && a.kind == 0 && haveK && haveV;

  // ---- keys: non-negative float bits of the (normalised) scores, -1 empty
  {
    const float divK = n_k > 0 ? fmaxf(tK / (float)n_k, kEps) : kEps;
    const float divV = n_v > 0 ? fmaxf(tV / (float)n_v, kEps) : kEps;
    for (int i = tid; i < nK + nV; i += kBlock) {
      float x = sc[i];
      int u = -1;
      if (x >= 0.f) {
        if (do_norm) x = i < nK ? (x / divK) * a.lam_k : (x / divV) * a.lam_v;
        u = (int)(__float_as_uint(x) & 0x7fffffffu);
      }
      key[i] = u;
    }
    __syncthreads();
  }

  // ---- how many of each kind (residual_router.py:305-365)
  int takeK = haveK ? min(bud_k, n_k) : 0, takeV = haveV ? min(bud_v, n_v) : 0;
  if (pol == 2) {
    // k_first: the K budget first; the rest of the joint allowance (the V
    // budget, the budgets being capped at the candidate counts) on the V
    // candidates scoring at least their mean
    takeV = 0;
    if (haveV) {
      float sv_loc = 0.f;
      for (int i = nK + tid; i < nK + nV; i += kBlock)
        if (key[i] >= 0) sv_loc += __int_as_float(key[i]);
      const float vmean = block_sum_fast(sv_loc, bs) / (float)n_v;
      int ge = 0;
      for (int i = nK + tid; i < nK + nV; i += kBlock) ge += key[i] >= 0 && __int_as_float(key[i]) >= vmean;
      takeV = min(bud_v, block_isum_fast(ge, bs));
    }
  } else if (pol == 3) {
    // adaptive: the joint allowance split by the attention entropy,
    // v_frac = H(max(a, 1e-6)) / log(max(N, 2))
    const int total = bud_k + bud_v;
    takeK = takeV = 0;
    if (total > 0) {
      const float* xq = a.xbuf + bq * a.Pmax * 16;
      float h = 0.f;
      int nt = 0;
      for (int i = tid; i < np * 16; i += kBlock) {
        const int nvp = A.valid[pg_base + (i >> 4)];
        if ((i & 15) >= nvp) continue;
        ++nt;
        float at = L > 0.f ? exp2_dn(xq[i] - M) : 0.f;
        at = a.pf ? (float)(_Float16)at : at / L;
        const float ac = fmaxf(at, kEps);
        h += ac * logf(ac);
      }
      const float ent = -block_sum_fast(h, bs);
      const int N = block_isum_fast(nt, bs);
      const double vfrac = fmin(1.0, fmax(0.0, (double)ent / log((double)max(N, 2))));
      const int v_alloc = max(0, (int)rint((double)total * vfrac));  // Python round: half to even
      const int k_alloc = max(0, total - v_alloc);
      takeK = want_k ? min(k_alloc, n_k) : 0;
      takeV = want_v ? min(v_alloc, n_v) : 0;
    }
  }

  // ---- thresholds and masks
  Sel sk{0u, 0, 0, false}, sv{0u, 0, 0, false};
  if (joint) {
    const int mb = min(bud_k + bud_v, n_k + n_v);
    sk = radix_select(key, 0, nK + nV, mb, hist, bs);
    sv = sk;
  } else {
    if (takeK > 0) sk = radix_select(key, 0, nK, takeK, hist, bs);
    if (takeV > 0) sv = radix_select(key, nK, nK + nV, takeV, hist, bs);
  }
  write_masks(key, maskq, np, k_cap, v_cap, nK, sk, sv, joint, 3, bs);

  // ---- read_budget_mode adaptive_score: per kind, keep the selected slots
  // whose score passes max(rel * top, abs) (top = the kind's best selected
  // score), or the best min_keep of them when fewer pass
  // (residual_router.py:366-410)
  if (a.adaptive_score) {
    for (int kind = 0; kind < 2; ++kind) {
      const int lo = kind == 0 ? 0 : nK, cap = kind == 0 ? k_cap : v_cap;
      float top = 0.f;
      int nsel = 0;
      for (int p = tid; p < np; p += kBlock) {
        const unsigned bits = kind == 0 ? (maskq[p] & 15u) : (maskq[p] >> 4);
        for (int r = 0; r < cap; ++r)
          if ((bits >> r) & 1u) {
            top = fmaxf(top, __int_as_float(key[lo + p * cap + r]));
            ++nsel;
          }
      }
      top = block_max_fast(top, bs);
      nsel = block_isum_fast(nsel, bs);
      if (nsel == 0) continue;
      auto passes = [&](float x) {
        return (a.rel_thr <= 0.0 || (double)x >= a.rel_thr * (double)top) &&
               (a.abs_thr <= 0.0 || (double)x >= a.abs_thr);
      };
      int kept = 0;
      for (int p = tid; p < np; p += kBlock) {
        const unsigned bits = kind == 0 ? (maskq[p] & 15u) : (maskq[p] >> 4);
        for (int r = 0; r < cap; ++r)
          if (((bits >> r) & 1u) && passes(__int_as_float(key[lo + p * cap + r]))) ++kept;
      }
      kept = block_isum_fast(kept, bs);
      if (a.min_keep > 0 && kept < a.min_keep) {
        // the best min_keep selected ones, ties in candidate order
        for (int p = tid; p < np; p += kBlock) {
          const unsigned bits = kind == 0 ? (maskq[p] & 15u) : (maskq[p] >> 4);
          for (int r = 0; r < cap; ++r)
            if (!((bits >> r) & 1u)) key[lo + p * cap + r] = -1;
        }
        __syncthreads();
        const Sel s2 = radix_select(key, lo, lo + np * cap, min(a.min_keep, nsel), hist, bs);
        const Sel off{0u, 0, 0, false};
        write_masks(key, maskq, np, k_cap, v_cap, nK, kind == 0 ? s2 : off, kind == 0 ? off : s2, false,
                    kind == 0 ? 1 : 2, bs);
      } else {
        for (int p = tid; p < np; p += kBlock) {
          unsigned m = maskq[p];
          for (int r = 0; r < cap; ++r) {
            const unsigned bit = 1u << (kind == 0 ? r : 4 + r);
            if ((m & bit) && !passes(__int_as_float(key[lo + p * cap + r]))) m &= ~bit;
          }
          maskq[p] = (uint8_t)m;
        }
      }
      __syncthreads();
    }
  }
  if (a.read_counts) {
    // ---- debug read counters: this query's selected K slots and V blocks
    // (each thread reads back the mask bytes it wrote)
    int ck = 0, cvb = 0;
    for (int p = tid; p < np; p += kBlock) {
      ck += __popc(maskq[p] & 15u);
      cvb += __popc((unsigned)maskq[p] >> 4);
    }
    ck = block_isum_fast(ck, bs);
    cvb = block_isum_fast(cvb, bs);
    if (tid == 0 && L > 0.f) {
      atomicAdd(a.read_counts, (unsigned long long)ck);
      atomicAdd(a.read_counts + 1, (unsigned long long)cvb);
      atomicAdd(a.read_counts + 2, 1ull);
    }
  }
  if (!diagp) return;
  // ---- diag: selected candidates in ascending candidate order (each
  // thread reads back the mask bytes it wrote)
  int sel_run = 0;
  for (int kind = 0; kind < 2; ++kind) {
    for (int p0 = 0; p0 < np; p0 += kBlock) {
      const int p = p0 + tid;
      const unsigned bits = p < np ? (kind == 0 ? (maskq[p] & 15u) : (maskq[p] >> 4)) : 0u;
      int tot;
      int pos = block_excl_scan(__popc(bits), bs, &tot) + sel_run;
      sel_run += tot;
      if (!bits) continue;
      const long pg = pg_base + p;
      const int cap = kind == 0 ? k_cap : v_cap;
      const int nsub = kind == 0 ? NCG : kVtb;
      int rr = 0;
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
  for (int i = sel_run + tid; i < a.diag_cap; i += kBlock) diagp[i] = -1;
}

// Wave-per-query form of decode_select_kernel<D, false, true> for rows of
// at most 256 pages (prompt rows of the prefill correction, short decode
// rows): one wave per query column, four columns per work-group and no
// barrier, where the work-group form spends most of a short row on its
// block reductions and four radix passes.  Lane l holds pages l + 64j.
// Every float sum is taken in the work-group form's order (a butterfly per
// 64 pages, then the four totals in page order), the k-th largest key comes
// from a binary search over its 31 bits, and ties at it are taken in
// candidate order, so the (M, L), masks and diag lists are the same bits.
// One K and one V candidate per page (k_cap = v_cap = 1), the joint or
// separate policy, no adaptive_score, correction on, the moments' K score.
template <int D>
__global__ __launch_bounds__(256) void decode_select_wave_kernel(carekv_arena A, DecodeArgs a) {
  constexpr int NCG = D / 32;
  constexpr int NJ = 4;  // pages per lane
  const int GQ = a.GQ, ngq = (GQ + 3) / 4;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the ngq work-groups of one (sequence, kv head) on one XCD, as in the
  // work-group form; prefill rows: the latest (longest) rows first
  const int win_d = blockIdx.x / (kXcd * ngq), rem = blockIdx.x % (kXcd * ngq);
  const int win = a.pf ? (int)(gridDim.x / (kXcd * ngq)) - 1 - win_d : win_d;
  const int pair = win * kXcd + rem % kXcd, qq = (rem / kXcd) * 4 + w;
  if (pair >= a.B * A.n_kv_heads || qq >= GQ) return;  // whole waves; no barrier follows
  const int kvh = pair % A.n_kv_heads, b = pair / A.n_kv_heads;
  const int bk = b * A.n_kv_heads + kvh;
  const EntryRow er = entry_row(A, a, b);
  const int np = er.np, seq = er.seq;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const long bq = (long)bk * GQ + qq;
  int32_t* diagp = nullptr;
  if (a.diag) {
    if (a.pf) {
      const PfCol x = pf_col(a, b, kvh, qq);
      diagp = x.ok ? a.diag + pf_row_off(a, x) * a.diag_cap : nullptr;
    } else {
      diagp = a.diag + ((long)b * a.Hq + kvh * GQ + qq) * a.diag_cap;
    }
  }
  // Lane l holds items l + 64j for j < nj (wave-uniform): a row's pages, or
  // the split partials; the slices j >= nj hold no item and are skipped (a
  // scalar branch), which changes no value: their keys are -1, their ballots
  // empty and their sums +0.
  const int njp = (np + 63) / 64;
  // sum of one value per (lane, j < nj) in the work-group form's order
  auto ordered_sum = [&](const float (&v)[NJ], int nj) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (j < nj) t = j == 0 ? wave_sum_f(v[0]) : t + wave_sum_f(v[j]);
    return t;
  };

  // ---- softmax statistics from the split partials (nsplit <= 256)
  const int nsr = splits_read(a, b);
  float mloc = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int s = lane + 64 * j;
    if (s < nsr) mloc = fmaxf(mloc, a.pml[(((long)bk * a.nsplit + s) * 16 + qq) * 2]);
  }
  const float M = wave_max_f(mloc);
  float lj[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    lj[j] = 0.f;
    const int s = lane + 64 * j;
    if (M != -INFINITY && s < nsr) {
      const long base = ((long)bk * a.nsplit + s) * 16 + qq;
      const float ms = a.pml[base * 2];
      if (ms != -INFINITY) lj[j] = a.pml[base * 2 + 1] * __builtin_amdgcn_exp2f(ms - M);
    }
  }
  const float L = ordered_sum(lj, (nsr + 63) / 64);
  if (lane == 0) { a.ml[bq * 2] = M; a.ml[bq * 2 + 1] = L; }

  // ---- one K and one V score per page (decode_select_kernel's K1 scoring)
  const float* recq = a.rec + bq * a.Pmax * a.F;
  const float invL = L > 0.f ? (a.pf ? 1.f : 1.f / L) : 0.f;
  const float* vsq_row = a.pf ? a.pf_vsq + (long)kvh * a.pf_pages : nullptr;
  const bool sens1 = a.sens_d == 1.0;
  float sK[NJ], sV[NJ];
  int cgK[NJ], vbV[NJ];
  int cntK = 0, cntV = 0;
  bool ovf = false;
  // Two page slices at a time: the loads of both are issued (every lane,
  // its page clamped to the row's last) before either is scored, so that a
  // lane waits one memory round trip per pair of slices, not per slice; the
  // scoring is the same arithmetic on the same values.
  struct PageIn {
    int nv, hm, ksl[NCG], vsl[kVtb];
    float vsq, r[7];
    uint2 e2;
  };
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    sK[j] = sV[j] = -1.f;
    cgK[j] = vbV[j] = -1;
  }
#pragma unroll
  for (int j0 = 0; j0 < NJ; j0 += 2) {
    if (j0 >= njp) break;
    PageIn in[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int pc = min(lane + 64 * (j0 + h), np - 1);
      const long pg = pg_base + pc;
      in[h].nv = A.valid[pg];
      in[h].hm = A.has_meta[pg];
      in[h].vsq = vsq_row ? vsq_row[pc] : A.v_sq[pg];
      load_slots<NCG>(in[h].ksl, A.k_slot + pg * NCG);
      load_slots<kVtb>(in[h].vsl, A.v_slot + pg * kVtb);
      in[h].e2 = *reinterpret_cast<const uint2*>(A.v_err + pg * kVtb);
      const float* rp = recq + (long)pc * 7;
#pragma unroll
      for (int k = 0; k < 7; ++k) in[h].r[k] = rp[k];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = j0 + h;
      const int p = lane + 64 * j;
      if (p >= np) continue;
      const int nv = in[h].nv, hm = in[h].hm;
      const float vsq = in[h].vsq;
      const int* ksl = in[h].ksl;
      const int* vsl = in[h].vsl;
      const uint2 e2 = in[h].e2;
      const float r0 = in[h].r[0], M2 = in[h].r[1], M3 = in[h].r[2], M4 = in[h].r[3], Ds = in[h].r[4],
                  es = in[h].r[5], E = in[h].r[6];
      const bool ok = L > 0.f && nv > 0 && hm;
      const float c = ok ? exp2_dn(r0 - M) * invL : 0.f;
      int nks = 0, nvs = 0, cg1 = -1, vb1 = -1;
#pragma unroll
      for (int cg = NCG - 1; cg >= 0; --cg)
        if (slot_ok(A, ksl[cg])) { ++nks; cg1 = cg; }
#pragma unroll
      for (int vb = kVtb - 1; vb >= 0; --vb)
        if (slot_ok(A, vsl[vb])) { ++nvs; vb1 = vb; }
      ovf |= hm && (nks > 1 || nvs > 1);
      cgK[j] = cg1;
      vbV[j] = vb1;
      if (ok && nks > 0) {
        const float wr = es * (1.f - c * es);
        const float q2 = (M2 - c * (2.f * M3 - c * M4)) + Ds * (wr * wr);
        float ks = kscore_underflows(c, M2, Ds, es) ? 0.f : (c * sqrt_dn(fmaxf(q2, 0.f))) * __builtin_amdgcn_sqrtf(vsq);
        if (!isfinite(ks)) ks = 0.f;
        sK[j] = ks * a.sens;
        ++cntK;
      }
      if (ok && vb1 >= 0 && vb1 * kVtb < nv) {
        const uint32_t ew = vb1 < 2 ? e2.x : e2.y;
        const float ve = h2f((uint16_t)(ew >> (16 * (vb1 & 1))));
        const float verr_s = sens1 ? ve : (float)((double)ve * a.sens_d);
        sV[j] = ((c * E) * verr_s) * a.sens;
        ++cntV;
      }
    }
  }
  if (a.pf && lane == 0) {  // the prompt's later pages: candidates that count, scored 0 (layer.py:514-517)
    const int* suf = a.pf_suf + (long)kvh * 3 * (a.pf_pages + 1);
    cntK += suf[np];
    cntV += suf[(a.pf_pages + 1) + np];
    ovf |= suf[2 * (a.pf_pages + 1) + np] != 0;
  }
  if (__any(ovf) && lane == 0) *a.err_flag = 1;
  float pk[NJ], pvv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) { pk[j] = sK[j] >= 0.f ? sK[j] : 0.f; pvv[j] = sV[j] >= 0.f ? sV[j] : 0.f; }
  const float tK = ordered_sum(pk, njp), tV = ordered_sum(pvv, njp);
  const int n_k = wave_sum_i(cntK), n_v = wave_sum_i(cntV);

  // ---- read budgets, normalisation, keys (as decode_select_kernel)
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
  const bool joint = a.policy == 1 && a.kind == 0 && haveK && haveV;
  const float divK = n_k > 0 ? fmaxf(tK / (float)n_k, kEps) : kEps;
  const float divV = n_v > 0 ? fmaxf(tV / (float)n_v, kEps) : kEps;
  int kK[NJ], kV[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float x = sK[j];
    kK[j] = -1;
    if (x >= 0.f) {
      if (do_norm) x = (x / divK) * a.lam_k;
      kK[j] = (int)(__float_as_uint(x) & 0x7fffffffu);
    }
    x = sV[j];
    kV[j] = -1;
    if (x >= 0.f) {
      if (do_norm) x = (x / divV) * a.lam_v;
      kV[j] = (int)(__float_as_uint(x) & 0x7fffffffu);
    }
  }

  // ---- thresholds: the k-th largest key of the K keys, the V keys or both
  // (keys -1: no candidate); every key taken when k reaches their count
  auto count_ge = [&](int t, bool useK, bool useV) {  // ballots: no cross-lane data movement
    int n = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j >= njp) break;
      if (useK) n += __builtin_popcountll(__ballot(kK[j] >= t));
      if (useV) n += __builtin_popcountll(__ballot(kV[j] >= t));
    }
    return n;
  };
  auto select = [&](int k, bool useK, bool useV) {
    Sel r{0u, INT_MAX, 0, true};
    if (count_ge(0, useK, useV) <= k) return r;
    uint32_t tau = 0u;
    for (int bit = 30; bit >= 0; --bit) {
      const uint32_t t = tau | (1u << bit);
      if (count_ge((int)t, useK, useV) >= k) tau = t;
    }
    r.tau = tau;
    r.take = k - count_ge((int)tau + 1, useK, useV);
    r.eq = count_ge((int)tau, useK, useV) - count_ge((int)tau + 1, useK, useV);
    return r;
  };
  const int takeK = haveK ? min(bud_k, n_k) : 0, takeV = haveV ? min(bud_v, n_v) : 0;
  Sel sk{0u, 0, 0, false}, sv{0u, 0, 0, false};
  if (joint) {
    sk = select(min(bud_k + bud_v, n_k + n_v), true, true);
    sv = sk;
  } else {
    if (takeK > 0) sk = select(takeK, true, false);
    if (takeV > 0) sv = select(takeV, false, true);
  }

  // ---- masks: keys above tau, ties at tau in candidate order (page order;
  // a joint selection's V ties after every K tie)
  const uint64_t below = (1ull << lane) - 1ull;
  int eq_runK = 0, eq_runV = 0;
  if (joint && sk.on && sk.take < sk.eq) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (j < njp) eq_runV += __builtin_popcountll(__ballot(kK[j] >= 0 && (uint32_t)kK[j] == sk.tau));
  }
  uint8_t* maskq = a.mask + bq * a.Pmax;
  unsigned selK[NJ], selV[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    selK[j] = selV[j] = 0u;
    if (j >= njp) continue;
    const int p = lane + 64 * j;
    const bool eqk = sk.on && kK[j] >= 0 && (uint32_t)kK[j] == sk.tau;
    const bool eqv = sv.on && kV[j] >= 0 && (uint32_t)kV[j] == sv.tau;
    const uint64_t bk_eq = __ballot(eqk), bv_eq = __ballot(eqv);
    const int rk = eq_runK + __builtin_popcountll(bk_eq & below);
    const int rv = eq_runV + __builtin_popcountll(bv_eq & below);
    eq_runK += __builtin_popcountll(bk_eq);
    eq_runV += __builtin_popcountll(bv_eq);
    bool tk = false, tv = false;
    if (sk.on && kK[j] >= 0) tk = (uint32_t)kK[j] > sk.tau || (eqk && rk < sk.take);
    if (sv.on && kV[j] >= 0) tv = (uint32_t)kV[j] > sv.tau || (eqv && rv < sv.take);
    selK[j] = tk ? 1u : 0u;
    selV[j] = tv ? 1u : 0u;
    if (p < np) maskq[p] = (uint8_t)(selK[j] | (selV[j] << 4));
  }
  if (a.read_counts) {
    int ck = 0, cvb = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) { ck += (int)selK[j]; cvb += (int)selV[j]; }
    ck = wave_sum_i(ck);
    cvb = wave_sum_i(cvb);
    if (lane == 0 && L > 0.f) {
      atomicAdd(a.read_counts, (unsigned long long)ck);
      atomicAdd(a.read_counts + 1, (unsigned long long)cvb);
      atomicAdd(a.read_counts + 2, 1ull);
    }
  }
  if (!diagp) return;
  // ---- diag: selected candidates in ascending candidate order (K then V)
  int run = 0;
  for (int kind = 0; kind < 2; ++kind) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j >= njp) break;
      const int p = lane + 64 * j;
      const bool on = kind == 0 ? selK[j] != 0u : selV[j] != 0u;
      const uint64_t bal = __ballot(on);
      const int pos = run + __builtin_popcountll(bal & below);
      run += __builtin_popcountll(bal);
      if (on && pos < a.diag_cap) diagp[pos] = (kind << 30) | (p << 3) | (kind == 0 ? cgK[j] : vbV[j]);
    }
  }
  for (int i = run + lane; i < a.diag_cap; i += 64) diagp[i] = -1;
}

int launch_decode_select(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  const int pairs = a.B * A.n_kv_heads;
  const dim3 grid(((pairs + kXcd - 1) / kXcd) * kXcd * a.GQ);
  const size_t lds = (a.correction && a.ncand <= kLdsCand) ? (size_t)a.ncand * sizeof(float) : 0;
  const bool px = a.correction && a.proxy;
  const bool k1 = a.k_cap == 1 && a.v_cap == 1;
  // rows of at most 256 pages with one K and one V slot, and enough query
  // columns to fill the GPU with waves (or short rows, where the work-group
  // form's fixed cost dominates): a wave per query.  CAREKV_SELECT_WAVE=0
  // keeps the work-group form, =2 takes the wave form for every row it covers.
  const char* env = getenv("CAREKV_SELECT_WAVE");
  const int wmode = env ? env[0] - '0' : 1;
  const long cols = (long)pairs * a.GQ;
  if (wmode != 0 && a.correction && !px && k1 && (a.policy == 0 || a.policy == 1) && !a.adaptive_score &&
      a.Pmax <= 256 && a.nsplit <= 256 && a.F == 7 && (wmode == 2 || cols >= 2048 || a.Pmax <= 64)) {
    const int ngq = (a.GQ + 3) / 4;
    const dim3 gw(((pairs + kXcd - 1) / kXcd) * kXcd * ngq);
    if (A.head_dim == 64) hipLaunchKernelGGL((decode_select_wave_kernel<64>), gw, dim3(kBlock), 0, s, A, a);
    else if (A.head_dim == 128) hipLaunchKernelGGL((decode_select_wave_kernel<128>), gw, dim3(kBlock), 0, s, A, a);
    else {
      set_error("unsupported head_dim %d", A.head_dim);
      return CAREKV_EINVAL;
    }
    CAREKV_CHECK_LAUNCH("decode_select (wave per query)");
    return CAREKV_OK;
  }
  const bool lc = lds > 0;
  auto go = [&](auto d, auto p, auto k, auto l) {
    hipLaunchKernelGGL((decode_select_kernel<decltype(d)::value, decltype(p)::value, decltype(k)::value,
                                             decltype(l)::value>),
                       grid, dim3(kBlock), lds, s, A, a);
  };
  using T = std::true_type;
  using F = std::false_type;
  auto by_lc = [&](auto d, auto p, auto k) {
    if (lc) go(d, p, k, T{});
    else go(d, p, k, F{});
  };
  auto by_kind = [&](auto d) {
    if (px) by_lc(d, T{}, F{});
    else if (k1) by_lc(d, F{}, T{});
    else by_lc(d, F{}, F{});
  };
  if (A.head_dim == 64) by_kind(std::integral_constant<int, 64>{});
  else if (A.head_dim == 128) by_kind(std::integral_constant<int, 128>{});
  else {
    set_error("unsupported head_dim %d", A.head_dim);
    return CAREKV_EINVAL;
  }
  CAREKV_CHECK_LAUNCH("decode_select");
  return CAREKV_OK;
}

}  // namespace carekv
