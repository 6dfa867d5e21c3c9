// Finalize pass of the CARE-KV decode: one work-group per (kv head,
// sequence), after the streaming kernel.  Combines the split partials into
// O_base, scores every stored slot (attention.py:704-790) from the page
// records, normalises per query (830-844), selects the joint or separate
// top-k with ties toward the lowest candidate index (856-875), and applies
// the exact softmax renormalisation (96-118) or the linear form (938-943)
// over the selected pages; writes half(O_base + dO).
#include "decode_common.h"
#include "host_util.h"

namespace carekv {

constexpr float kEps = 1e-6f;       // residual_router.py:34
constexpr int kMaxItems = 512;      // apply work-list chunk


// ------------------------------------------------------------ block helpers
// Exclusive prefix count of `flag` over the 256 threads; total in *total.
__device__ __forceinline__ int block_excl_count(bool flag, int* wsum, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned long long m = __ballot(flag);
  const int in_wave = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) wsum[w] = __popcll(m);
  __syncthreads();
  int before = 0;
  for (int i = 0; i < w; ++i) before += wsum[i];
  *total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  __syncthreads();
  return before + in_wave;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  // deterministic fixed-order tree
  red[threadIdx.x] = v;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

struct Seg {
  const float* p;
  int n;        // entries
  int base;     // global candidate index of entry 0
  int norm;
  float div, lam;
};

__device__ __forceinline__ float seg_val(const Seg& s, int i) {
  float x = s.p[i];
  if (!(x >= 0.f)) return -1.f;              // empty candidate position
  if (s.norm) x = (x / s.div) * s.lam;
  return x;
}

// k-th largest over the valid entries of up to two segments: returns the
// threshold bit pattern and how many entries equal to it are taken (lowest
// candidate index first).  Non-negative floats order like their bits.
__device__ void radix_select(const Seg* sg, int nseg, int k, uint32_t* tau, int* take_eq, int* hist, int* bc) {
  uint32_t prefix = 0, mask = 0;
  int krem = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int s = 0; s < nseg; ++s)
      for (int i = threadIdx.x; i < sg[s].n; i += 256) {
        const float v = seg_val(sg[s], i);
        if (v < 0.f) continue;
        const uint32_t u = __float_as_uint(v);
        if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
      }
    __syncthreads();
    if (threadIdx.x == 0) {
      int cum = 0, d = 255;
      for (; d > 0; --d) {
        if (cum + hist[d] >= krem) break;
        cum += hist[d];
      }
      bc[0] = (int)(prefix | ((uint32_t)d << shift));
      bc[1] = krem - cum;
    }
    __syncthreads();
    prefix = (uint32_t)bc[0];
    krem = bc[1];
    mask |= 255u << shift;
    __syncthreads();
  }
  *tau = prefix;
  *take_eq = krem;
}

// Append the selected global candidate indices (ascending) to out[*count..].
__device__ void select_write(const Seg* sg, int nseg, uint32_t tau, int take_eq, int32_t* out, int* count,
                             int* wsum, int* bc) {
  if (threadIdx.x == 0) { bc[2] = 0; bc[3] = *count; }
  __syncthreads();
  for (int s = 0; s < nseg; ++s)
    for (int base = 0; base < sg[s].n; base += 256) {
      const int i = base + threadIdx.x;
      const float v = i < sg[s].n ? seg_val(sg[s], i) : -1.f;
      const uint32_t u = __float_as_uint(v);
      const bool gt = v >= 0.f && u > tau, eq = v >= 0.f && u == tau;
      int tot_eq;
      const int r_eq = block_excl_count(eq, wsum, &tot_eq) + bc[2];
      const bool take = gt || (eq && r_eq < take_eq);
      int tot_sel;
      const int pos = block_excl_count(take, wsum, &tot_sel) + bc[3];
      if (take) out[pos] = sg[s].base + i;
      __syncthreads();
      if (threadIdx.x == 0) { bc[2] += tot_eq; bc[3] += tot_sel; }
      __syncthreads();
    }
  if (threadIdx.x == 0) *count = bc[3];
  __syncthreads();
}

// ================================================================ phase 2
// One work-group per (sequence, kv head), launched after the streaming
// kernel on the same stream (the kernel boundary orders its writes).
template <int D, int BITS>
__global__ __launch_bounds__(256) void decode_finalize_kernel(carekv_arena A, DecodeArgs a) {
  constexpr int RB = row_bytes(D, BITS);
  constexpr int NCG = D / 32;
  constexpr int KSB = kPage * 32 / 2;
  constexpr int VSB = kVtb * D / 2;
  __shared__ __align__(16) char smem[16 * D * 4 + 2048 + 64];
  __shared__ int s_misc[16];
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int Hkv = A.n_kv_heads, GQ = a.GQ;
  const int bk = b * Hkv + kvh;
  const int seq_raw = a.seq_slot[b], np_raw = a.n_pages[b];
  const bool row_ok = seq_raw >= 0 && seq_raw < A.n_seq && np_raw >= 0 && np_raw <= a.Pmax;
  const int seq = row_ok ? seq_raw : 0, np = row_ok ? np_raw : 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const int F = a.F;
  float* s_ob = reinterpret_cast<float*>(smem);            // [16][D] O_base
  float* s_red = s_ob + 16 * D;                             // [256]
  int* hist = reinterpret_cast<int*>(s_red + 256);          // [256]
  int* wsum = hist + 256;                                   // [4]
  int* bc = wsum + 4;                                       // [8]
  __shared__ float s_M[16], s_L[16], s_nk[16], s_nv[16];
  __shared__ int s_item_page[kMaxItems];
  __shared__ unsigned char s_item_km[kMaxItems], s_item_vm[kMaxItems];
  __shared__ int s_ent_page[kMaxItems];
  __shared__ unsigned char s_ent_sub[kMaxItems], s_ent_kind[kMaxItems];
  __shared__ float s_num[4][D], s_den[4];

  // ---- combine splits
  for (int idx = threadIdx.x; idx < GQ * D; idx += 256) {
    const int qq = idx / D, d = idx % D;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.pml[(((long)bk * a.nsplit + s) * 16 + qq) * 2]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
      for (int s = 0; s < a.nsplit; ++s) {
        const long base = ((long)bk * a.nsplit + s) * 16 + qq;
        const float ms = a.pml[base * 2];
        if (ms == -INFINITY) continue;
        const float f = expf(ms - M);
        L += a.pml[base * 2 + 1] * f;
        O += a.po[base * D + d] * f;
      }
    }
    s_ob[qq * D + d] = L > 0.f ? O / L : 0.f;
    if (d == 0) { s_M[qq] = M; s_L[qq] = L; }
  }
  __syncthreads();
  const bool empty = !(s_L[0] > 0.f);
  uint16_t* outp = a.out + ((long)b * a.Hq + kvh * GQ) * D;
  int32_t* diagp = a.diag ? a.diag + ((long)b * a.Hq + kvh * GQ) * a.diag_cap : nullptr;
  auto write_base_out = [&]() {
    for (int idx = threadIdx.x; idx < GQ * D; idx += 256) outp[idx] = f2h(s_ob[idx]);
    if (diagp)
      for (int idx = threadIdx.x; idx < GQ * a.diag_cap; idx += 256) diagp[idx] = -1;
  };
  if (!a.correction || empty) { write_base_out(); return; }

  // ---- score every stored slot (candidate index = page*cap + rank)
  const int nK = np * a.k_cap, nV = np * a.v_cap;
  float sumK[16], sumV[16];
#pragma unroll
  for (int qq = 0; qq < 16; ++qq) sumK[qq] = sumV[qq] = 0.f;
  int cntK = 0, cntV = 0;
  float* scb = a.scores + (long)bk * GQ * a.ncand;
  for (int p = threadIdx.x; p < np; p += 256) {
    const long pg = pg_base + p;
    const int nv = A.valid[pg];
    const bool ok = nv > 0 && A.has_meta[pg];
    int ksl[NCG], vsl[kVtb];
#pragma unroll
    for (int c = 0; c < NCG; ++c) ksl[c] = ok ? A.k_slot[pg * NCG + c] : -1;
#pragma unroll
    for (int v = 0; v < kVtb; ++v) vsl[v] = ok ? A.v_slot[pg * kVtb + v] : -1;
    const float vnorm = sqrtf(A.v_sq[pg]);
    float verr_s[kVtb];
#pragma unroll
    for (int v = 0; v < kVtb; ++v) verr_s[v] = (float)((double)h2f(A.v_err[pg * kVtb + v]) * a.sens_d);
    const float* recp = a.rec + ((long)bk * a.Pmax + p) * GQ * F;
    for (int qq = 0; qq < GQ; ++qq) {
      const float* r = recp + qq * F;
      const float c = ok ? expf(r[0] - s_M[qq]) / s_L[qq] : 0.f;
      float* sk = scb + (long)qq * a.ncand + p * a.k_cap;
      float* sv = scb + (long)qq * a.ncand + nK + p * a.v_cap;
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        if (ksl[cg] < 0 || rk >= a.k_cap) continue;
        const float M2 = r[1 + 3 * rk], M3 = r[2 + 3 * rk], M4 = r[3 + 3 * rk];
        const float q2 = c * c * (M2 - c * (2.f * M3 - c * M4));
        float ks = sqrtf(fmaxf(q2, 0.f)) * vnorm;
        if (!isfinite(ks)) ks = 0.f;
        ks = ks * a.sens;
        sk[rk] = ks;
        sumK[qq] += ks;
        cntK += qq == 0;
        ++rk;
      }
      for (; rk < a.k_cap; ++rk) sk[rk] = -1.f;
      int rv = 0;
#pragma unroll
      for (int vb = 0; vb < kVtb; ++vb) {
        if (vsl[vb] < 0 || rv >= a.v_cap) continue;
        float vsc = -1.f;
        if (vb * kVtb < nv) {
          vsc = (c * r[1 + 3 * a.k_cap + rv]) * verr_s[vb];
          vsc = vsc * a.sens;
          sumV[qq] += vsc;
          cntV += qq == 0;
        }
        sv[rv] = vsc;
        ++rv;
      }
      for (; rv < a.v_cap; ++rv) sv[rv] = -1.f;
    }
  }
  // deterministic reductions
  const float nkf = block_sum((float)cntK, s_red), nvf = block_sum((float)cntV, s_red);
  const int n_k = (int)nkf, n_v = (int)nvf;
  for (int qq = 0; qq < GQ; ++qq) {
    const float tk = block_sum(sumK[qq], s_red), tv = block_sum(sumV[qq], s_red);
    if (threadIdx.x == 0) {
      s_nk[qq] = n_k > 0 ? fmaxf(tk / (float)n_k, kEps) : kEps;
      s_nv[qq] = n_v > 0 ? fmaxf(tv / (float)n_v, kEps) : kEps;
    }
  }
  // ---- read budgets (residual_router.py:37-76 via attention.py:662-670)
  const bool want_k = (a.kind == 0 || a.kind == 1) && n_k > 0;
  const bool want_v = (a.kind == 0 || a.kind == 2) && n_v > 0;
  const int tk = want_k ? n_k : 0, tv = want_v ? n_v : 0;
  int bud_k, bud_v;
  if (!a.budget_ratio) {
    bud_k = a.abs_k; bud_v = a.abs_v;
  } else {
    bud_k = (a.ratio_k > 0.0 && tk > 0) ? max(1, (int)((double)tk * a.ratio_k)) : 0;
    bud_v = (a.ratio_v > 0.0 && tv > 0) ? max(1, (int)((double)tv * a.ratio_v)) : 0;
  }
  if (a.kind == 2) bud_k = 0;
  if (a.kind == 1) bud_v = 0;
  bud_k = min(bud_k, tk);
  bud_v = min(bud_v, tv);
  const bool haveK = want_k && bud_k > 0, haveV = want_v && bud_v > 0;
  __syncthreads();
  if (!haveK && !haveV) { write_base_out(); return; }
  const bool do_norm = a.normalize && a.kind == 0 && haveK && haveV;
  const bool joint = a.joint && a.kind == 0 && haveK && haveV;

  for (int qq = 0; qq < GQ; ++qq) {
    // ---- selection
    const float* base_q = scb + (long)qq * a.ncand;
    Seg sk{base_q, nK, 0, do_norm, s_nk[qq], a.lam_k};
    Seg sv{base_q + nK, nV, nK, do_norm, s_nv[qq], a.lam_v};
    int32_t* selq = a.sel + ((long)bk * GQ + qq) * a.ncand;
    __shared__ int s_nsel;
    if (threadIdx.x == 0) s_nsel = 0;
    __syncthreads();
    uint32_t tau;
    int take;
    if (joint) {
      int mb = (bud_k > 0 && bud_v > 0) ? bud_k + bud_v : max(bud_k, bud_v);
      mb = min(mb, n_k + n_v);
      Seg two[2] = {sk, sv};
      radix_select(two, 2, mb, &tau, &take, hist, bc);
      select_write(two, 2, tau, take, selq, &s_nsel, wsum, bc);
    } else {
      if (haveK) {
        radix_select(&sk, 1, min(bud_k, n_k), &tau, &take, hist, bc);
        select_write(&sk, 1, tau, take, selq, &s_nsel, wsum, bc);
      }
      if (haveV) {
        radix_select(&sv, 1, min(bud_v, n_v), &tau, &take, hist, bc);
        select_write(&sv, 1, tau, take, selq, &s_nsel, wsum, bc);
      }
    }
    const int nsel = s_nsel;
    __syncthreads();

    // ---- apply over the selected pages, in chunks of kMaxItems entries
    float num[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) num[c] = 0.f;
    float den = 0.f;
    constexpr int NGL = D / 32;                // lanes per token in the apply
    const int at = lane / NGL, ag = lane % NGL; // token, channel group
    const bool alane = at < kPage;
    const float qscale = a.sm_scale;
    float qf[32];
    {
      const uint16_t* qp = a.q + ((long)b * a.Hq + kvh * GQ + qq) * D + ag * 32;
#pragma unroll
      for (int c = 0; c < 32; ++c) qf[c] = alane ? h2f(qp[c]) : 0.f;
    }
    const float Mq = s_M[qq], Lq = s_L[qq];
    for (int e0 = 0; e0 < nsel; e0 += kMaxItems) {
      const int ne = min(kMaxItems, nsel - e0);
      // decode entries in parallel: (kind, page, sub)
      for (int i = threadIdx.x; i < ne; i += 256) {
        const int gidx = selq[e0 + i];
        int kind, page, rank;
        if (gidx < nK) { kind = 0; page = gidx / a.k_cap; rank = gidx % a.k_cap; }
        else { kind = 1; page = (gidx - nK) / a.v_cap; rank = (gidx - nK) % a.v_cap; }
        const long pg = pg_base + page;
        int sub = 0, r = 0;
        if (kind == 0) {
          for (int c = 0; c < NCG; ++c) if (A.k_slot[pg * NCG + c] >= 0) { if (r == rank) { sub = c; break; } ++r; }
        } else {
          for (int v = 0; v < kVtb; ++v) if (A.v_slot[pg * kVtb + v] >= 0) { if (r == rank) { sub = v; break; } ++r; }
        }
        s_ent_page[i] = page; s_ent_sub[i] = (unsigned char)sub; s_ent_kind[i] = (unsigned char)kind;
        if (diagp && e0 + i < a.diag_cap) diagp[(long)qq * a.diag_cap + e0 + i] = (kind << 30) | (page << 3) | sub;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        // merge the page-sorted K entries and V entries into page items
        int nk_e = 0;
        while (nk_e < ne && s_ent_kind[nk_e] == 0) ++nk_e;
        int i = 0, j = nk_e, n_it = 0;
        while (i < nk_e || j < ne) {
          int pg_i = i < nk_e ? s_ent_page[i] : 0x7fffffff;
          int pg_j = j < ne ? s_ent_page[j] : 0x7fffffff;
          const int pgn = min(pg_i, pg_j);
          unsigned char km = 0, vm = 0;
          while (i < nk_e && s_ent_page[i] == pgn) km |= (unsigned char)(1u << s_ent_sub[i++]);
          while (j < ne && s_ent_page[j] == pgn) vm |= (unsigned char)(1u << s_ent_sub[j++]);
          s_item_page[n_it] = pgn; s_item_km[n_it] = km; s_item_vm[n_it] = vm; ++n_it;
        }
        s_misc[1] = n_it;
      }
      __syncthreads();
      const int n_it = s_misc[1];
      for (int it = w; it < n_it; it += 4) {
        const int page = s_item_page[it];
        const unsigned km = s_item_km[it], vm = s_item_vm[it];
        const long pg = pg_base + page;
        const int nv = A.valid[pg];
        if (!alane || at >= nv) continue;
        // logit of token at (recomputed from the cache)
        uint32_t kw2[BITS], vw2[BITS];
        load_bytes<4 * BITS>(kw2, A.kcodes + (pg * kPage + at) * RB + ag * 4 * BITS);
        _Float16 ks, vs;
        if (A.scale_mode == 1) {
          ks = (_Float16)((float)((const int8_t*)A.kscale)[(pg * kPage + at) * NCG + ag] * h2f(A.kmaster[pg]));
          vs = (_Float16)((float)((const int8_t*)A.vscale)[(pg * kPage + at) * NCG + ag] * h2f(A.vmaster[pg]));
        } else {
          ks = bits2half(((const uint16_t*)A.kscale)[(pg * kPage + at) * NCG + ag]);
          vs = bits2half(((const uint16_t*)A.vscale)[(pg * kPage + at) * NCG + ag]);
        }
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < 32; ++c) dot += (float)dq(get_code<BITS>(kw2, c), ks) * qf[c];
        float wk = 0.f;
        if (km & (1u << ag)) {
          const int slot = A.k_slot[pg * NCG + ag];
          const long so2 = (long)seq * A.n_slots + slot;
          uint32_t rw[4];
          load_bytes<16>(rw, A.k_res + so2 * KSB + at * 16);
          const float rs = h2f(A.k_res_scale[so2]);
#pragma unroll
          for (int c = 0; c < 32; ++c) wk += qf[c] * ((float)get_code<4>(rw, c) * rs);
        }
#pragma unroll
        for (int o = 1; o < NGL; o <<= 1) {
          dot += __shfl_xor(dot, o, 64);
          wk += __shfl_xor(wk, o, 64);
        }
        const float At = expf(dot * qscale - Mq) / Lq;
        const int vb = at / kVtb;
        const bool vsel = (vm >> vb) & 1u;
        float coefK = 0.f, coefV = 0.f;
        if (a.k_exact) {
          const float ds = wk / a.sqrt_d;
          if (km) { coefK = At * expm1f(ds); if (ag == 0) den += coefK; }
          if (vsel) coefV = At * expf(ds);
        } else {
          if (km) coefK = a.k_corr_scale * At * wk;
          if (vsel) coefV = At;
        }
        if (km) {
          load_bytes<4 * BITS>(vw2, A.vcodes + (pg * kPage + at) * RB + ag * 4 * BITS);
#pragma unroll
          for (int c = 0; c < 32; ++c) {
            const float vh = (float)dq(get_code<BITS>(vw2, c), vs);
            num[c] += coefK * (a.k_exact ? vh : vh - s_ob[qq * D + ag * 32 + c]);
          }
        }
        if (vsel) {
          const int slot = A.v_slot[pg * kVtb + vb];
          const long so2 = (long)seq * A.n_slots + slot;
          uint32_t rw[4];
          load_bytes<16>(rw, A.v_res + so2 * VSB + (at - vb * kVtb) * (D / 2) + ag * 16);
          const float rs = h2f(A.v_res_scale[so2]);
#pragma unroll
          for (int c = 0; c < 32; ++c) num[c] += coefV * ((float)get_code<4>(rw, c) * rs);
        }
      }
      __syncthreads();
    }
    // ---- reduce num over tokens (lanes with equal ag) and waves
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      float v = num[c];
#pragma unroll
      for (int o = NGL; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
      num[c] = v;
    }
    den = wave_sum(den);
    if (lane < NGL) {
#pragma unroll
      for (int c = 0; c < 32; ++c) s_num[w][lane * 32 + c] = num[c];
    }
    if (lane == 0) s_den[w] = den;
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += 256) {
      const float nm = s_num[0][d] + s_num[1][d] + s_num[2][d] + s_num[3][d];
      const float dn = s_den[0] + s_den[1] + s_den[2] + s_den[3];
      const float ob = s_ob[qq * D + d];
      const float o = a.k_exact ? (ob + nm) / (1.f + dn) : ob + nm;
      outp[qq * D + d] = f2h(o);
    }
    if (diagp)
      for (int i = nsel + threadIdx.x; i < a.diag_cap; i += 256) diagp[(long)qq * a.diag_cap + i] = -1;
    __syncthreads();
  }
}


int launch_decode_finalize(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto bb) {
    hipLaunchKernelGGL((decode_finalize_kernel<decltype(d)::value, decltype(bb)::value>), dim3(A.n_kv_heads, a.B),
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_finalize");
    return CAREKV_OK;
  });
}

}  // namespace carekv
