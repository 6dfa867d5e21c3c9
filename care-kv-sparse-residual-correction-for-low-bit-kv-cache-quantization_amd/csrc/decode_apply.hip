// Apply pass of the CARE-KV decode: one work-group per (page chunk, kv
// head, sequence), after the select kernel.  Every page of the chunk that
// any query of the GQA group selected a slot of is processed once for all
// the group's queries, a wave per page, with the per-query masks:
//
//   a_t   = e_t 2^(m_ref - M)              (unnormalised attention weight, e_t
//                                            stored by the streaming pass)
//   dS_t  = sum over selected K slots of q_cg . R_K[t] (raw, residual scale)
//   exact mode (attention.py:96-118 in closed form; with sum_t A_t = 1):
//     num += sum_t a_t (e^{dS_t/sqrt(D)} - 1) V_hat_t
//          + sum_{t in selected V blocks} a_t e^{dS_t/sqrt(D)} R_V[t]
//     den += sum_t a_t (e^{dS_t/sqrt(D)} - 1)
//     out  = (O_base + num / L) / (1 + den / L)
//   linear mode (attention.py:938-943):
//     num += k_corr_scale * sum_t a_t dS_t V_hat_t + sum_{sel V} a_t R_V[t]
//     den += k_corr_scale * sum_t a_t dS_t
//     out  = O_base + (num - den * O_base) / L
// Both products run on MFMA like the streaming pass (V_hat / R_V transposed
// through LDS), with each weight split into fp16 hi + lo halves: the
// correction terms can be large against O_base (wide V rows, large dS) and
// partly cancel, so fp16 weights alone cost several output ulps.  The
// combine kernel sums the chunk partials in chunk order and writes half(out).
#include "block_util.h"
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

template <int D, int BITS>
constexpr bool same_slot_order() {
  using G = PageGeom<D, BITS>;
  for (int i = 0; i < G::CH; ++i)
    if (G::PB::T.slot_code[i] != G::PR::T.slot_code[i]) return false;
  return true;
}

// One page of the apply pass as loaded ahead of its use.
template <int D, int BITS>
struct ApplyItem {
  static constexpr int NWC = PageGeom<D, BITS>::NWC, NCG = D / 32, CH = D / 4;
  int p;               // page (wave-uniform)
  int meta;            // page metadata, one field per lane
  unsigned mk;         // selection mask byte of this lane's query (ln)
  unsigned kany, vany; // slots selected by any query of the group (wave-uniform)
  uint32_t e01, e23;   // e of tokens 4j..4j+3 for query ln, fp16 pairs
  float mref;          // m_ref of query ln at the page
  uint32_t vw[NWC];    // V codes of token ln, chunk lj (when a K slot is selected)
  uint32_t vsc;        // its scale code
  uint32_t kr[NCG];    // K residual word of each stored slot (cg order) that is selected
  uint32_t krs[NCG];   // and its scale (fp16 bits: converted where the item is used, since a
                       // conversion at the load would wait for it and for every load before it)
  uint32_t rv[CH / 8]; // V residual chunk of tile row ln (when its block is selected)
  uint32_t rvs;        // and its scale (fp16 bits)
  bool rsel;           // tile row ln holds a selected V block
};

// 4 waves per SIMD (2 for the fp16 base, whose rows take twice the
// registers): the register budget is capped at 128 (256) VGPRs.
template <int D, int BITS, int SM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BITS == 16 ? 2 : 4, 8)))
void decode_apply_kernel(carekv_arena A, DecodeArgs a) {
  using G = PageGeom<D, BITS>;
  using Item = ApplyItem<D, BITS>;
  static_assert(same_slot_order<D, BITS>(), "V residual tile must use the V_hat slot order");
  constexpr int NT = G::NT, NCG = G::NCG, CH = G::CH, CHB = G::CHB, RB = G::RB;
  constexpr int VT_WORDS = kPage * G::VROW;
  constexpr int MERGE_BYTES = 4 * 16 * (D / 2) * 4;
  constexpr int TILE_BYTES = 4 * VT_WORDS * 4;
  constexpr int LDS_BYTES = MERGE_BYTES > TILE_BYTES ? MERGE_BYTES : TILE_BYTES;
  constexpr int kMaxSP = 1024;
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ __align__(16) _Float16 sq[16 * D];
  __shared__ __align__(16) _Float16 sqr[16 * D];
  __shared__ int s_items[kMaxSP];
  __shared__ float s_den[4][16];
  __shared__ BlockScratch bs;

  // prefill rows: the latest (longest) rows first
  const int chunk = blockIdx.x, kvh = blockIdx.y, b = a.pf ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const EntryRow er = entry_row(A, a, b);
  const int seq = er.seq, np = er.np;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  RowRes rr;
  if (BITS == 16 && a.pf) {  // prefill rows: the prompt's dense fp16 K_hat / V_hat
    const long off = (long)kvh * a.pf_T * D;  // rows past the prompt read as 0
    const uint32_t bytes = (uint32_t)a.pf_T * D * 2;
    rr.kc = make_rsrc(a.pf_k + off, bytes);
    rr.vc = make_rsrc(a.pf_v + off, bytes);
    rr.ks = make_rsrc(nullptr, 0u);
    rr.vs = make_rsrc(nullptr, 0u);
  } else {
    rr = row_resources<D, BITS, SM>(A, pg_base);
  }
  const uint8_t* maskb = a.mask + (long)bk * GQ * a.Pmax;
  const bool exact = a.k_exact != 0;
  const bool qv = ln < GQ;
  const long qrow = (long)bk * GQ + (qv ? ln : 0);  // this lane's query row of the workspace

  // ---- pages of the chunk with any selected slot
  int p_lo, p_hi;
  launch_pages(A, a, seq, np, p_lo, p_hi);
  const int p_begin = p_lo + chunk * a.SPA, p_end = min(p_begin + a.SPA, p_hi);
  int n_items = 0;
  for (int p0 = p_begin; p0 < p_end; p0 += kBlock) {
    const int p = p0 + threadIdx.x;
    unsigned any = 0;
    if (p < p_end)
      for (int n = 0; n < GQ; ++n) any |= maskb[(long)n * a.Pmax + p];
    int tot;
    const int pos = block_excl_scan(any ? 1 : 0, bs, &tot);
    if (any) s_items[n_items + pos] = p;
    n_items += tot;
  }
  if (a.pf) {
    stage_q_by<D>(sq, sqr, [&](int n) {
      const PfCol x = pf_col(a, b, kvh, n);
      return x.ok ? a.q + pf_row_off(a, x) * D : (const uint16_t*)nullptr;
    });
  } else {
    stage_q<D>(sq, sqr, a.q + ((long)b * a.Hq + kvh * GQ) * D, GQ);
  }
  __syncthreads();

  const float Mq = qv ? a.ml[qrow * 2] : 0.f;
  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * VT_WORDS;
  float4_t nacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) nacc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  float den = 0.f;

  // e^x - 1 and e^x from the hardware base-2 exponential; a short series
  // keeps e^x - 1 accurate for the small |x| of residual logit shifts.
  auto em1 = [](float x) {
    if (fabsf(x) < 0.03125f) return x * (1.f + x * (0.5f + x * (0.16666667f + x * 0.041666668f)));
    return __builtin_amdgcn_exp2f(x * 1.44269504f) - 1.f;
  };
  // The tile rows a page leaves unwritten keep finite data from earlier
  // pages and meet zero weights; start from zeros.
  for (int i = lane; i < VT_WORDS; i += 64) vt[i] = 0u;
  lds_sync_wave();

  // Two-stage prefetch: the metadata and masks of item it + 8, and the data
  // of item it + 4 (issued with that item's metadata already at hand).
  struct MStage { int p, meta; unsigned mk; };
  auto load_m = [&](int it) {
    MStage m;
    m.p = __builtin_amdgcn_readfirstlane(s_items[it]);
    m.meta = meta_lanes_load<NCG>(A, pg_base + m.p, lane);
    m.mk = qv ? maskb[(long)ln * a.Pmax + m.p] : 0u;
    return m;
  };
  auto load_d = [&](const MStage& m, Item& d) {
    d.p = m.p; d.meta = m.meta; d.mk = m.mk;
    const PageMeta<NCG> pm = meta_from_lanes<NCG>(m.meta, A);
    const unsigned kb = m.mk & 15u, vb = m.mk >> 4;
    d.kany = 0; d.vany = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (__any((kb >> r) & 1u)) d.kany |= 1u << r;
      if (__any((vb >> r) & 1u)) d.vany |= 1u << r;
    }
    d.e01 = 0u; d.e23 = 0u; d.mref = 0.f;
    if (qv) {
      const uint2 e = *reinterpret_cast<const uint2*>(a.ebuf + (qrow * a.Pmax + m.p) * 16 + 4 * lj);
      d.e01 = e.x; d.e23 = e.y;
      d.mref = a.rec[(qrow * a.Pmax + m.p) * a.F];
    }
    if (d.kany) {
      const uint32_t vrow = (uint32_t)(m.p * kPage + ln);
      buf_load<CHB>(d.vw, rr.vc, vrow * RB + lj * CHB);
      const int gi = (lj * CH) / 32;
      if constexpr (SM == 1) d.vsc = __builtin_amdgcn_raw_buffer_load_b8(rr.vs, vrow * NCG + gi, 0, 0);
      else d.vsc = __builtin_amdgcn_raw_buffer_load_b16(rr.vs, (vrow * NCG + gi) * 2, 0, 0);
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        d.kr[cg] = 0u; d.krs[cg] = 0u;
        if (pm.ksl[cg] < 0) continue;
        if (rk < a.k_cap && ((d.kany >> rk) & 1u)) {
          const long so = (long)seq * A.n_slots + pm.ksl[cg];
          const __amdgpu_buffer_rsrc_t r = make_rsrc(A.k_res + so * G::KSB, G::KSB);
          d.kr[cg] = __builtin_amdgcn_raw_buffer_load_b32(r, ln * 16 + lj * 4, 0, 0);
          d.krs[cg] = A.k_res_scale[so];
        }
        ++rk;
      }
    }
    d.rsel = false;
    if (d.vany) {
      // tile row ln: block ln / 4, token ln % 4 of that block's slot
      const int vb_row = ln >> 2;
      int rrank = -1, rslot = -1, r2 = 0;
#pragma unroll
      for (int v = 0; v < kVtb; ++v) {
        if (pm.vsl[v] < 0) continue;
        if (v == vb_row) { rrank = r2; rslot = pm.vsl[v]; }
        ++r2;
      }
      d.rsel = rrank >= 0 && rrank < a.v_cap && ((d.vany >> rrank) & 1u) && 4 * vb_row < pm.nv;
      if (d.rsel) {
        const long so = (long)seq * A.n_slots + rslot;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(A.v_res + so * G::VSB, G::VSB);
        buf_load<CH / 2>(d.rv, r, (ln & 3) * (D / 2) + lj * (CH / 2));
        d.rvs = A.v_res_scale[so];
      }
    }
  };

  MStage mB{}, mC{};
  Item cur, nxt;
  if (w < n_items) {
    const MStage m0 = load_m(w);
    if (w + 4 < n_items) mB = load_m(w + 4);
    load_d(m0, nxt);
  }
  for (int it = w; it < n_items; it += 4) {
    cur = nxt;
    if (it + 8 < n_items) mC = load_m(it + 8);
    if (it + 4 < n_items) load_d(mB, nxt);
    mB = mC;

    const PageMeta<NCG> cm = meta_from_lanes<NCG>(cur.meta, A);
    const unsigned kbits = cur.mk & 15u, vbits = cur.mk >> 4;
    // ---- attention weights of the page: a_t = e_t 2^(m_ref - M)
    float at[4];
    {
      const float f = qv ? __builtin_amdgcn_exp2f(cur.mref - Mq) : 0.f;
      half2_t e01, e23;
      __builtin_memcpy(&e01, &cur.e01, 4);
      __builtin_memcpy(&e23, &cur.e23, 4);
      at[0] = (float)e01[0] * f; at[1] = (float)e01[1] * f;
      at[2] = (float)e23[0] * f; at[3] = (float)e23[1] * f;
    }
    // ---- dS over the K slots this lane's query selected
    float wk[4] = {0.f, 0.f, 0.f, 0.f};
    if (cur.kany) {
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        if (cm.ksl[cg] < 0) continue;
        if (rk >= a.k_cap) break;
        if ((cur.kany >> rk) & 1u) {
          const float4_t racc = kslot_dot_w(cur.kr[cg], sqr, D, cg, ln, lj);
          const float rs = ((kbits >> rk) & 1u) ? h2f((uint16_t)cur.krs[cg]) : 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) wk[i] = fmaf(racc[i], rs, wk[i]);
        }
        ++rk;
      }
    }
    // ---- V block of this lane's tokens (4j .. 4j+3): stored slot rank
    int vrank = -1, rv = 0;
#pragma unroll
    for (int vb = 0; vb < kVtb; ++vb) {
      if (cm.vsl[vb] < 0) continue;
      if (vb == lj) vrank = rv;
      ++rv;
    }
    const bool vsel = vrank >= 0 && vrank < a.v_cap && ((vbits >> vrank) & 1u);
    float ck[4], cv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (exact) {
        const float m1 = em1(wk[i] * a.inv_sqrt_d);
        ck[i] = kbits ? at[i] * m1 : 0.f;
        cv[i] = vsel ? at[i] * (1.f + m1) : 0.f;
      } else {
        ck[i] = kbits ? a.k_corr_scale * at[i] * wk[i] : 0.f;
        cv[i] = vsel ? at[i] : 0.f;
      }
    }
    den += (ck[0] + ck[1]) + (ck[2] + ck[3]);
    // ---- num += ck V_hat
    if (cur.kany) {
      float vm = 0.f;
      if constexpr (SM == 1) vm = h2f((uint16_t)cm.vmaster);
      const _Float16 vs = lane_scale<SM>(SM == 1 ? (int)(int8_t)cur.vsc : (int)cur.vsc, vm);
      half2_t vp[CH / 2];
      dequant_pairs<BITS, CH, BITS>(cur.vw, vs, vp);
      vtile_write<D, BITS>(vt, vp, ln, lj);
      half4_t ah, al;
      split_weights(ck, ah, al);
      lds_sync_wave();
      pv_accumulate2<D, BITS>(vt, ah, al, nacc, ln, lj);
      lds_sync_wave();
    }
    // ---- num += cv R_V over the V blocks some query selected; the other
    // rows keep finite data and meet zero weights
    if (cur.vany) {
      if (cur.rsel) {
        half2_t rp[CH / 2];
        dequant_pairs<4, CH, BITS>(cur.rv, bits2half((uint16_t)cur.rvs), rp);
        vtile_write<D, BITS>(vt, rp, ln, lj);
      }
      half4_t ah, al;
      split_weights(cv, ah, al);
      lds_sync_wave();
      pv_accumulate2<D, BITS>(vt, ah, al, nacc, ln, lj);
      lds_sync_wave();
    }
  }

  // ---- merge the waves and write the chunk partial
  den = col_sum(den);
  if (lj == 0) s_den[w][ln] = den;
  const long cbase = ((long)bk * a.nsplit + a.chunk_base + chunk) * GQ;
  sum_waves<D, BITS>(reinterpret_cast<float*>(smem), nacc, w, ln, lj, GQ, a.num + cbase * D);
  if ((int)threadIdx.x < GQ) {
    const int qq = threadIdx.x;
    a.den[cbase + qq] = ((s_den[0][qq] + s_den[1][qq]) + s_den[2][qq]) + s_den[3][qq];
  }
}

// out = half(O_base + correction): O_base from the split partials of the
// streaming pass, the correction from the chunk partials of the apply pass
// (both summed in a fixed order; O_base as O + po 2^(m_s - M), the product
// and the sum rounded apart, as the select kernel forms it without a
// correction).
// A thread takes 4 consecutive dims of one query; every load of its splits
// and chunks is issued before the sums that use it (batches of SB splits and
// CB chunks, indices clamped to the last one, read whatever L is), so a wave
// waits about one memory latency per batch instead of one per split.  The
// host sizes the batches to the counts (8 / 2 / 1 splits, 4 / 2 / 1 chunks),
// so that a call with one split does not issue seven clamped repeats.
template <int SB, int CB>
__global__ __launch_bounds__(256) void decode_combine_kernel(int Hkv, int D, int out_al8, DecodeArgs a) {
  const int D4 = D >> 2, GQ = a.GQ;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)a.B * Hkv * GQ * D4) return;
  const int d = (int)(gid % D4) * 4;
  const long r = gid / D4;
  const int qq = (int)(r % GQ), bk = (int)(r / GQ);
  const int b = bk / Hkv, kvh = bk % Hkv;
  long orow = (long)b * a.Hq + kvh * GQ + qq;
  if (a.pf) {  // prefill rows: the column's (row, head); padding columns write nothing
    const PfCol x = pf_col(a, b, kvh, qq);
    if (!x.ok) return;
    orow = pf_row_off(a, x);
  }
  const long bq = (long)bk * GQ + qq;
  const float M = a.ml[bq * 2], L = a.ml[bq * 2 + 1];
  const int ns = a.nsplit, nsr = splits_read(a, b), na = a.napply;
  const long sb = (long)bk * ns * 16 + qq;   // split s: row sb + 16 s of po / pml
  const long cb0 = (long)bk * ns * GQ + qq;  // chunk c: row cb0 + c GQ of num / den
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f), nm = make_float4(0.f, 0.f, 0.f, 0.f);
  float dn = 0.f;
  const int nb = max((nsr + SB - 1) / SB, (na + CB - 1) / CB);
  for (int k = 0; k < nb; ++k) {  // batch k: splits SB k .. SB k + SB-1 and chunks CB k .. CB k + CB-1
    float ms[SB], dv[CB];
    float4 pv[SB], nv[CB];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const long base = sb + 16L * min(SB * k + j, nsr - 1);
      ms[j] = a.pml[base * 2];
      pv[j] = *reinterpret_cast<const float4*>(a.po + base * D + d);
    }
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const long cb = cb0 + (long)max(min(CB * k + j, na - 1), 0) * GQ;
      nv[j] = *reinterpret_cast<const float4*>(a.num + cb * D + d);
      dv[j] = a.den[cb];
    }
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const float e = __builtin_amdgcn_exp2f(ms[j] - M);
      if (SB * k + j < nsr && ms[j] != -INFINITY) {  // product and sum rounded apart (no contraction)
        O.x += pv[j].x * e;
        O.y += pv[j].y * e;
        O.z += pv[j].z * e;
        O.w += pv[j].w * e;
      }
    }
#pragma unroll
    for (int j = 0; j < CB; ++j) {  // chunks past the last add +0, which leaves a sum begun at +0 unchanged
      const bool in = CB * k + j < na;
      nm.x += in ? nv[j].x : 0.f;
      nm.y += in ? nv[j].y : 0.f;
      nm.z += in ? nv[j].z : 0.f;
      nm.w += in ? nv[j].w : 0.f;
      dn += in ? dv[j] : 0.f;
    }
  }
  auto fin = [&](float Oc, float nmc) -> uint32_t {
    const float ob = L > 0.f ? Oc / L : 0.f;
    float o = ob;
    if (L > 0.f) {
      if (a.k_exact) {
        o = (ob + nmc / L) / (1.f + dn / L);
      } else if (a.pf) {
        // prefill rows: the reference adds the linear terms to its
        // unnormalised fp16-weight O_base (layer.py:553-557)
        o = Oc + (nmc - dn * Oc);
      } else {
        o = ob + (nmc - dn * ob) / L;
      }
    }
    return f2h(o);
  };
  const uint32_t h0 = fin(O.x, nm.x), h1 = fin(O.y, nm.y), h2 = fin(O.z, nm.z), h3 = fin(O.w, nm.w);
  uint16_t* op = a.out + orow * D + d;
  if (out_al8) {
    *reinterpret_cast<uint2*>(op) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
  } else {
    op[0] = (uint16_t)h0;
    op[1] = (uint16_t)h1;
    op[2] = (uint16_t)h2;
    op[3] = (uint16_t)h3;
  }
}

int launch_decode_apply(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  if (a.SPA > 1024) {
    set_error("apply chunks must be at most 1024 pages");
    return CAREKV_EINVAL;
  }
  if (!a.pf && A.base_bits != 16 && a.GQ <= 4)
    return launch_decode_apply4(A, a, s);  // windows of 4 pages, 4x4x4 layout
  const dim3 grid(a.napply_run, A.n_kv_heads, a.B);
  // prefill rows read the prompt's fp16 K_hat / V_hat whatever the cache base
  const int bits = a.pf ? 16 : A.base_bits, smode = a.pf ? 0 : A.scale_mode;
  return dispatch_dbs16(A.head_dim, bits, smode, [&](auto d, auto bb, auto sm) {
    hipLaunchKernelGGL((decode_apply_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value>), grid,
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_apply");
    return CAREKV_OK;
  });
}

int launch_decode_combine(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  if (A.head_dim % 4 != 0) {
    set_error("decode_combine: head_dim %d is not a multiple of 4", A.head_dim);
    return CAREKV_EINVAL;
  }
  const long n = (long)a.B * A.n_kv_heads * a.GQ * (A.head_dim / 4);
  if (n == 0) return CAREKV_OK;
  const int out_al8 = (reinterpret_cast<uintptr_t>(a.out) & 7) == 0;
  const dim3 grid((unsigned)((n + 255) / 256));
  const int sb = a.nsplit >= 8 ? 8 : a.nsplit >= 2 ? 2 : 1, cb = a.napply >= 4 ? 4 : a.napply >= 2 ? 2 : 1;
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, A.n_kv_heads, A.head_dim, out_al8, a); };
  if (sb == 8) {
    if (cb == 4) go(decode_combine_kernel<8, 4>);
    else if (cb == 2) go(decode_combine_kernel<8, 2>);
    else go(decode_combine_kernel<8, 1>);
  } else if (sb == 2) {
    if (cb == 4) go(decode_combine_kernel<2, 4>);
    else if (cb == 2) go(decode_combine_kernel<2, 2>);
    else go(decode_combine_kernel<2, 1>);
  } else {
    if (cb == 4) go(decode_combine_kernel<1, 4>);
    else if (cb == 2) go(decode_combine_kernel<1, 2>);
    else go(decode_combine_kernel<1, 1>);
  }
  CAREKV_CHECK_LAUNCH("decode_combine");
  return CAREKV_OK;
}

}  // namespace carekv
