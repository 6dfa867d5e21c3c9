// Apply pass for GQA groups of at most 4 query heads (same inputs and
// outputs as decode_apply.hip): one work-group per (page chunk, kv head,
// sequence); each wave takes windows of 4 selected pages.
//
// Per window, in the layout of the 4x4x4 streaming pass (lane l: page
// l / 16 of the window, tokens 4*((l%16)/4) .. +3, query head l % 4):
//   * a_t = e_t 2^(m_ref - M) from the weights the streaming pass stored;
//   * dS_t = sum over the K slots the lane's query selected of
//     q_cg . R_K[t] * scale, on v_mfma_f32_4x4x4_16b_f16 (one residual row
//     per lane);
//   * the exact (attention.py:96-118) or linear (attention.py:938-943)
//     weights of V_hat and of the selected V residual rows.
// Then O-sized partials through the LDS tile, num^T += V^T c^T on 4x4x4
// blocks (A from the tile by the transpose load), which keeps only the 4
// query heads in the accumulator:
//   * num += ck V_hat for each page of the window with a selected K slot;
//   * num += cv R_V for the selected V blocks of the window, 4 blocks per
//     tile, dequantised by all 64 lanes.
// den accumulates the K weights; decode_combine_kernel finishes.
// With 2-bit bases (HL) each weight runs as fp16 hi + lo halves, as in
// decode_apply.hip: their logit shifts dS are large (up to ~5 with the KIVI
// base) and the weighted rows partly cancel against O_base, where fp16
// weights alone cost up to a few hundredths at |O| ~ 1.
//
// The loop is a software pipeline: the pages, metadata and mask bytes of a
// window are read two windows ahead, and each load that depends on them
// (stored weights, K residual rows, V codes, the first 4 V residual blocks)
// is issued for the next window as soon as the current window is done with
// the registers it lands in.  Every prefetch is issued by every lane (a lane
// with nothing to fetch reads out of range of a buffer resource, which
// returns 0 without a memory access, or a mapped stand-in it then drops), so
// the in-order load counter never waits across a branch.
#include "block_util.h"
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

// K1: at most one stored K slot and one stored V block per page (k_cap =
// v_cap = 1, the common store budget): the page's slot and block come from
// two ballots over the metadata lanes instead of the per-rank searches.
template <int D, int BITS, int SM, bool K1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void decode_apply4_kernel(carekv_arena A, DecodeArgs a) {
  using G = PageGeom<D, BITS>;
  using PR = Pairs<4, 32, 4>;  // pair schedule of a K residual row
  constexpr int NCG = G::NCG, CH = G::CH, CHB = G::CHB, RB = G::RB, NWC = G::NWC;
  constexpr bool HL = BITS == 2;  // weights as fp16 hi + lo
  constexpr int VT_WORDS = kPage * G::VROW;
  constexpr int MERGE_BYTES = 4 * 4 * D * 4;  // [wave][query][D] fp32
  constexpr int TILE_BYTES = 4 * VT_WORDS * 4;
  constexpr int LDS_BYTES = MERGE_BYTES > TILE_BYTES ? MERGE_BYTES : TILE_BYTES;
  constexpr int kMaxSP = 1024;
  constexpr uint32_t kOut = 0x80000000u;  // an out-of-range buffer offset
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ __align__(16) _Float16 sqr4[NCG * 8 * 16];  // [cg][step][query][4]: q in the residual order
  __shared__ int s_items[kMaxSP];
  __shared__ float s_den[4][4];
  __shared__ __align__(16) uint2 s_pk[4][64], s_pv[4][64];  // per wave: [page][query][token group] ck, cv
  __shared__ __align__(16) uint2 s_pkl[HL ? 4 : 1][64], s_pvl[HL ? 4 : 1][64];  // HL: their lo halves
  __shared__ int s_blk[4][2][16];  // per wave and window parity: selected V blocks, (4 pi + vb) | slot << 4
  __shared__ BlockScratch bs;

  // prefill rows: the latest (longest) rows first
  const int chunk = blockIdx.x, kvh = blockIdx.y, b = a.pf ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const int seq_raw = a.seq_slot[b], np_raw = a.n_pages[b];
  const bool row_ok = seq_raw >= 0 && seq_raw < A.n_seq && np_raw >= 0 && np_raw <= a.Pmax;
  const int seq = row_ok ? seq_raw : 0, np = row_ok ? np_raw : 0;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;  // V side: token/row ln, chunk lj; S side: page lj of the window
  const int sc = lane & 3, sbk = ln >> 2;    // S side: query sc, tokens 4*sbk.. (V block sbk)
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const RowRes rr = row_resources<D, BITS, SM>(A, pg_base);
  const __amdgpu_buffer_rsrc_t kres = make_rsrc(A.k_res + (long)seq * A.n_slots * G::KSB, (uint32_t)A.n_slots * G::KSB);
  const __amdgpu_buffer_rsrc_t vres = make_rsrc(A.v_res + (long)seq * A.n_slots * G::VSB, (uint32_t)A.n_slots * G::VSB);
  const uint16_t* kres_s = A.k_res_scale + (long)seq * A.n_slots;
  const uint16_t* vres_s = A.v_res_scale + (long)seq * A.n_slots;
  const uint8_t* maskb = a.mask + (long)bk * GQ * a.Pmax;
  const bool exact = a.k_exact != 0;
  const bool qv = sc < GQ;
  const long qrow = (long)bk * GQ + (qv ? sc : 0);  // this lane's query row of the workspace

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
  {  // q in the residual MFMA order
    const uint16_t* qg = a.q + ((long)b * a.Hq + kvh * GQ) * D;
    for (int i = threadIdx.x; i < NCG * 128; i += 256) {
      const int cg = i >> 7, s = (i >> 4) & 7, c = (i >> 2) & 3, e = i & 3;
      sqr4[i] = c < GQ ? bits2half(qg[c * D + cg * 32 + PR::T.slot_code[4 * s + e]]) : (_Float16)0.f;
    }
  }
  __syncthreads();

  const float Mq = qv ? a.ml[qrow * 2] : 0.f;
  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * VT_WORDS;
  float4_t nacc[D / 64];  // num[query sc][slots 64h + 4(lane/4) .. +3]
#pragma unroll
  for (int h = 0; h < D / 64; ++h) nacc[h] = float4_t{0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  // Tile rows a pass leaves unwritten keep finite data and meet zero weights.
  for (int i = lane; i < VT_WORDS; i += 64) vt[i] = 0u;
  lds_sync_wave();

  auto em1 = [](float x) {  // e^x - 1, a short series for the small |x| of residual logit shifts
    if (fabsf(x) < 0.03125f) return x * (1.f + x * (0.5f + x * (0.16666667f + x * 0.041666668f)));
    return __builtin_amdgcn_exp2f(x * 1.44269504f) - 1.f;
  };

  // ---- pipeline stages
  // page (S side: page lj), its metadata field ln, the lane's mask byte.
  // load_pre issues the raw loads (the field's aligned word, the mask byte)
  // and finish_pre, one window later, turns them into the field and the
  // mask, so that no wait for them falls in the window that issued them.
  struct WinPre { int page, meta; unsigned mk; };
  auto load_pre = [&](int base) {
    WinPre x;
    const int it = base + lj;
    x.page = it < n_items ? s_items[min(it, kMaxSP - 1)] : -1;
    const int pc = x.page >= 0 ? x.page : 0;
    x.meta = (int)meta_word_load<NCG, SM>(A, pg_base + pc, ln);
    x.mk = maskb[(long)(qv ? sc : 0) * a.Pmax + pc];
    return x;
  };
  auto finish_pre = [&](WinPre& x) {
    const bool ok = x.page >= 0;
    const long pg = pg_base + (ok ? x.page : 0);
    x.meta = ok ? meta_word_field<NCG, SM>(A, (uint32_t)x.meta, pg, ln) : 0;
    x.mk = (ok && qv) ? x.mk : 0u;
  };
  // uniform digest of a window: pages, which slot ranks any query selected
  struct Plan { int pg[4]; unsigned kany[4], vany[4]; int nblk; };
  auto make_plan = [&](const WinPre& x, int par) {
    Plan p;
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      p.pg[pi] = __builtin_amdgcn_readlane(x.page, 16 * pi);
      p.kany[pi] = 0u;
      p.vany[pi] = 0u;
    }
    const unsigned kbits = x.mk & 15u, vbits = x.mk >> 4;
#pragma unroll
    for (int r = 0; r < (K1 ? 1 : 4); ++r) {
      const unsigned long long kb = __ballot((kbits >> r) & 1u), vb = __ballot((vbits >> r) & 1u);
#pragma unroll
      for (int pi = 0; pi < 4; ++pi) {
        if ((kb >> (16 * pi)) & 0xffffull) p.kany[pi] |= 1u << r;
        if ((vb >> (16 * pi)) & 0xffffull) p.vany[pi] |= 1u << r;
      }
    }
    // selected V blocks in (page, block) order: lane l stands for block
    // bb = l % 16 (page bb / 4, V block bb % 4); its rank among the page's
    // stored blocks decides whether a query selected it
    const int bb = lane & 15, bpi = bb >> 2;
    const int s = __shfl(x.meta, 16 * bpi + 6 + (bb & 3), 64);
    const bool stored = s >= 0 && s < A.n_slots;
    const unsigned sm = (unsigned)(__ballot(stored) & 0xffffull);
    const int rank = __builtin_popcount(sm & (0xfu << (4 * bpi)) & ((1u << bb) - 1u));
    const unsigned va = bpi == 0 ? p.vany[0] : bpi == 1 ? p.vany[1] : bpi == 2 ? p.vany[2] : p.vany[3];
    const bool sel = stored && rank < a.v_cap && ((va >> rank) & 1u);
    const unsigned selm = (unsigned)(__ballot(sel) & 0xffffull);
    p.nblk = __builtin_popcount(selm);
    if (lane < 16 && sel) s_blk[w][par][__builtin_popcount(selm & ((1u << bb) - 1u))] = bb | (s << 4);
    return p;
  };
  // stored weights and m_ref of the lane's (page, query)
  struct WinE { uint32_t e01, e23; float mref; };
  auto load_e = [&](const WinPre& x) {
    WinE e;
    const long r = qrow * a.Pmax + (x.page >= 0 ? x.page : 0);
    const uint2 v = *reinterpret_cast<const uint2*>(a.ebuf + r * 16 + 4 * sbk);
    e.e01 = v.x; e.e23 = v.y;
    e.mref = a.rec[r * a.F];
    return e;
  };
  // K1: the first stored K channel group (-1: none) and the first stored V
  // block of the lane's page lj, from ballots over its metadata lanes
  struct First { int cg, slot, vb; };
  auto first_slots = [&](const WinPre& x) {
    First f;
    const int fld = lane & 15;
    const bool in_arena = x.meta >= 0 && x.meta < A.n_slots;
    const unsigned long long kb = __ballot(fld >= 2 && fld < 2 + NCG && in_arena);
    const unsigned long long vb = __ballot(fld >= 6 && fld < 6 + kVtb && in_arena);
    const uint32_t km = (uint32_t)(kb >> (16 * lj + 2)) & ((1u << NCG) - 1u);
    const uint32_t vm = (uint32_t)(vb >> (16 * lj + 6)) & 0xfu;
    f.cg = km ? (int)__builtin_ctz(km) : -1;
    f.vb = vm ? (int)__builtin_ctz(vm) : -1;
    f.slot = __shfl(x.meta, (lane & 48) + 2 + (km ? (int)__builtin_ctz(km) : 0), 64);
    return f;
  };
  // K residual row ln of the lowest selected rank of the lane's page lj
  struct KRow { uint32_t w[4]; float scale; int rank; };
  auto load_krow = [&](const WinPre& x, const Plan& p) {
    KRow k;
    const unsigned ka = lj == 0 ? p.kany[0] : lj == 1 ? p.kany[1] : lj == 2 ? p.kany[2] : p.kany[3];
    const int r0 = ka ? __builtin_ctz(ka) : -1;
    int slot = -1, cnt = 0;
    if constexpr (K1) {
      const First f = first_slots(x);
      slot = (r0 == 0 && f.cg >= 0) ? f.slot : -1;
    } else {
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int s = __shfl(x.meta, (lane & 48) + 2 + cg, 64);
        if (s < 0 || s >= A.n_slots) continue;
        if (cnt == r0) slot = s;
        ++cnt;
      }
    }
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(kres, slot >= 0 ? (uint32_t)slot * G::KSB + ln * 16 : kOut, 0, 0);
    k.w[0] = v[0]; k.w[1] = v[1]; k.w[2] = v[2]; k.w[3] = v[3];
    k.scale = h2f(kres_s[slot >= 0 ? slot : 0]);
    k.rank = slot >= 0 ? r0 : -1;
    return k;
  };
  // V codes and scales (V side: token ln, chunk lj) of the pages with a
  // selected K slot
  struct VCodes { uint32_t vw[4][NWC]; uint32_t vsc[4]; };
  auto load_vcodes = [&](const Plan& p) {
    VCodes v;
    const int gi = (lj * CH) / 32;
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      const bool on = p.kany[pi] != 0u;
      const uint32_t vrow = (uint32_t)(max(p.pg[pi], 0) * kPage + ln);
      buf_load<CHB>(v.vw[pi], rr.vc, on ? vrow * RB + lj * CHB : kOut);
      if constexpr (SM == 1) v.vsc[pi] = __builtin_amdgcn_raw_buffer_load_b8(rr.vs, on ? vrow * NCG + gi : kOut, 0, 0);
      else v.vsc[pi] = __builtin_amdgcn_raw_buffer_load_b16(rr.vs, on ? (vrow * NCG + gi) * 2 : kOut, 0, 0);
    }
    return v;
  };
  // V residual rows of blocks r0 .. r0+3 of the list (lane l: block
  // r0 + l / 16, row (l % 16) / 4, chunk l % 4)
  struct VRes { uint32_t w[CH / 8]; float scale; };
  auto load_vres = [&](int par, int r0, int nblk) {
    VRes v;
    const int k = r0 + lj;
    const int e = s_blk[w][par][min(k, 15)];
    const bool on = k < nblk;
    const int slot = on ? (e >> 4) : 0;
    const int m = ln >> 2, c = ln & 3;
    buf_load<CH / 2>(v.w, vres, on ? (uint32_t)slot * G::VSB + m * (D / 2) + c * (CH / 2) : kOut);
    v.scale = h2f(vres_s[slot]);
    return v;
  };

  // ---- prologue: window 0 resolved, window 1's page records in flight
  int base = 4 * w, par = 0;
  WinPre pre0 = load_pre(base), pre1 = load_pre(base + 16);
  finish_pre(pre0);
  Plan plan0 = make_plan(pre0, 0);
  WinE e0 = load_e(pre0);
  KRow kr0 = load_krow(pre0, plan0);
  VCodes vc0 = load_vcodes(plan0);
  VRes vr0 = load_vres(0, 0, plan0.nblk);

  for (; base < n_items; base += 16, par ^= 1) {
    const WinPre cur = pre0;
    const Plan cp = plan0;
    const WinE ce = e0;
    pre0 = pre1;
    pre1 = load_pre(base + 32);
    finish_pre(pre0);
    plan0 = make_plan(pre0, par ^ 1);
    e0 = load_e(pre0);

    const unsigned kbits = cur.mk & 15u, vbits = cur.mk >> 4;
    const int my_nv = __shfl(cur.meta, lane & 48, 64);
    const unsigned kany_all = cp.kany[0] | cp.kany[1] | cp.kany[2] | cp.kany[3];

    // ---- attention weights a_t = e_t 2^(m_ref - M)
    float at[4];
    {
      const float f = qv ? __builtin_amdgcn_exp2f(ce.mref - Mq) : 0.f;
      half2_t e01, e23;
      __builtin_memcpy(&e01, &ce.e01, 4);
      __builtin_memcpy(&e23, &ce.e23, 4);
      at[0] = (float)e01[0] * f; at[1] = (float)e01[1] * f;
      at[2] = (float)e23[0] * f; at[3] = (float)e23[1] * f;
    }

    // ---- dS over the selected K slots (rank r: r-th stored slot of the page)
    float wk[4] = {0.f, 0.f, 0.f, 0.f};
    First cf{-1, -1, -1};
    if constexpr (K1) cf = first_slots(cur);
    if constexpr (K1) {
      // the page's one stored K slot, its row prefetched by load_krow
      const unsigned ka = lj == 0 ? cp.kany[0] : lj == 1 ? cp.kany[1] : lj == 2 ? cp.kany[2] : cp.kany[3];
      if (kany_all & 1u) {
        const bool need = cf.cg >= 0 && (ka & 1u);
        const int cgq = cf.cg >= 0 ? cf.cg : 0;
        float4_t racc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const half2_t c0 = code_pair<4, 32, 4>(kr0.w, 2 * s);
          const half2_t c1 = code_pair<4, 32, 4>(kr0.w, 2 * s + 1);
          const half4_t ar = {c0[0], c0[1], c1[0], c1[1]};
          const half4_t bq = *reinterpret_cast<const half4_t*>(sqr4 + ((cgq * 8 + s) * 4 + sc) * 4);
          racc = mfma4x4(ar, bq, racc);
        }
        const float use = (need && (kbits & 1u)) ? kr0.scale : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) wk[i] = fmaf(racc[i], use, wk[i]);
      }
    } else {
      int kslot[NCG];
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int s = __shfl(cur.meta, (lane & 48) + 2 + cg, 64);
        kslot[cg] = (s >= 0 && s < A.n_slots) ? s : -1;
      }
      const unsigned ka = lj == 0 ? cp.kany[0] : lj == 1 ? cp.kany[1] : lj == 2 ? cp.kany[2] : cp.kany[3];
      for (int r = 0; r < a.k_cap && r < NCG; ++r) {
        if (!((kany_all >> r) & 1u)) continue;
        int cgr = -1, slotr = -1, cnt = 0;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          if (kslot[cg] < 0) continue;
          if (cnt == r) { cgr = cg; slotr = kslot[cg]; }
          ++cnt;
        }
        // rows are needed for pages where some query selected rank r
        const bool need = cgr >= 0 && ((ka >> r) & 1u);
        uint32_t rw[4] = {kr0.w[0], kr0.w[1], kr0.w[2], kr0.w[3]};
        float rs = kr0.scale;
        const bool fetch = need && r != kr0.rank;
        if (__any(fetch)) {  // a rank past the prefetched one (rare)
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(kres, fetch ? (uint32_t)slotr * G::KSB + ln * 16 : kOut, 0, 0);
          const float fs = h2f(kres_s[fetch ? slotr : 0]);
          if (fetch) {
            rw[0] = v[0]; rw[1] = v[1]; rw[2] = v[2]; rw[3] = v[3];
            rs = fs;
          }
        }
        const int cgq = cgr >= 0 ? cgr : 0;
        float4_t racc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const half2_t c0 = code_pair<4, 32, 4>(rw, 2 * s);
          const half2_t c1 = code_pair<4, 32, 4>(rw, 2 * s + 1);
          const half4_t ar = {c0[0], c0[1], c1[0], c1[1]};
          const half4_t bq = *reinterpret_cast<const half4_t*>(sqr4 + ((cgq * 8 + s) * 4 + sc) * 4);
          racc = mfma4x4(ar, bq, racc);
        }
        // the S-side lane (page lj, query sc) takes rank r if its query selected it
        const float use = (need && ((kbits >> r) & 1u)) ? rs : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) wk[i] = fmaf(racc[i], use, wk[i]);
      }
    }
    kr0 = load_krow(pre0, plan0);

    // ---- weights of V_hat (ck) and of the V residual rows (cv)
    int vrank = -1, rvn = 0;
    if constexpr (K1) {
      vrank = sbk == cf.vb ? 0 : -1;  // later stored blocks rank past v_cap
    } else {
#pragma unroll
      for (int v = 0; v < kVtb; ++v) {
        const int s = __shfl(cur.meta, (lane & 48) + 6 + v, 64);
        if (s < 0 || s >= A.n_slots) continue;
        if (v == sbk) vrank = rvn;
        ++rvn;
      }
    }
    const bool vsel = vrank >= 0 && vrank < a.v_cap && ((vbits >> vrank) & 1u) && 4 * sbk < my_nv;
    float ck[4], cv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (exact) {
        const float m1 = kbits ? em1(wk[i] * a.inv_sqrt_d) : 0.f;
        ck[i] = kbits ? at[i] * m1 : 0.f;
        cv[i] = vsel ? at[i] * (1.f + m1) : 0.f;
      } else {
        ck[i] = kbits ? a.k_corr_scale * at[i] * wk[i] : 0.f;
        cv[i] = vsel ? at[i] : 0.f;
      }
    }
    den += (ck[0] + ck[1]) + (ck[2] + ck[3]);
    const half2_t ck01 = {(_Float16)ck[0], (_Float16)ck[1]}, ck23 = {(_Float16)ck[2], (_Float16)ck[3]};
    const half2_t cv01 = {(_Float16)cv[0], (_Float16)cv[1]}, cv23 = {(_Float16)cv[2], (_Float16)cv[3]};
    pw_store_strided(s_pk[w], h2bits(ck01), h2bits(ck23), lane);
    pw_store(s_pv[w], h2bits(cv01), h2bits(cv23), lane);
    if constexpr (HL) {
      const half2_t kl01 = {(_Float16)(ck[0] - (float)ck01[0]), (_Float16)(ck[1] - (float)ck01[1])};
      const half2_t kl23 = {(_Float16)(ck[2] - (float)ck23[0]), (_Float16)(ck[3] - (float)ck23[1])};
      const half2_t vl01 = {(_Float16)(cv[0] - (float)cv01[0]), (_Float16)(cv[1] - (float)cv01[1])};
      const half2_t vl23 = {(_Float16)(cv[2] - (float)cv23[0]), (_Float16)(cv[3] - (float)cv23[1])};
      pw_store_strided(s_pkl[w], h2bits(kl01), h2bits(kl23), lane);
      pw_store(s_pvl[w], h2bits(vl01), h2bits(vl23), lane);
    }

    // ---- num += ck V_hat, page by page
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      if (!cp.kany[pi]) continue;
      _Float16 vs;
      if constexpr (SM == 1) {
        const float vm = h2f((uint16_t)__builtin_amdgcn_readlane(cur.meta, 16 * pi + 11));
        vs = (_Float16)((float)(int8_t)vc0.vsc[pi] * vm);
      } else {
        vs = bits2half((uint16_t)vc0.vsc[pi]);
      }
      half2_t vp[CH / 2];
      dequant_pairs<BITS, CH, BITS>(vc0.vw[pi], vs, vp);
      vtile_write<D, BITS>(vt, vp, ln, lj);
      lds_sync_wave();
      uint2 pg[4];  // ck[query sc][tokens g, g+4, g+8, g+12] of page pi
      pw_load(s_pk[w], pi, sc, pg);
#pragma unroll
      for (int g = 0; g < 4; ++g) pv4_group<D, BITS>(vt, g, pg[g].x, pg[g].y, nacc, lane);
      if constexpr (HL) {
        pw_load(s_pkl[w], pi, sc, pg);
#pragma unroll
        for (int g = 0; g < 4; ++g) pv4_group<D, BITS>(vt, g, pg[g].x, pg[g].y, nacc, lane);
      }
      lds_sync_wave();
    }

    vc0 = load_vcodes(plan0);

    // ---- num += cv R_V: the window's selected V blocks, 4 per tile (block
    // u of a round fills tile rows u, u+4, u+8, u+12); round 0 was prefetched
    for (int r0 = 0; r0 < cp.nblk; r0 += 4) {
      const VRes rv = r0 == 0 ? vr0 : load_vres(par, r0, cp.nblk);
      if (r0 + lj < cp.nblk) {
        const int m = ln >> 2, c = ln & 3;
        half2_t rp[CH / 2];
        dequant_pairs<4, CH, BITS>(rv.w, (_Float16)rv.scale, rp);
        vtile_write<D, BITS>(vt, rp, lj + 4 * m, c);
      }
      lds_sync_wave();
      // block r0 + u: cv[query sc][its 4 tokens] from S lane 16*pi_u + 4*vb_u + sc
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (r0 + u >= cp.nblk) break;
        const int bu = s_blk[w][par][r0 + u] & 15;
        const uint2 pu = s_pv[w][((bu >> 2) * 4 + sc) * 4 + (bu & 3)];
        pv4_group<D, BITS>(vt, u, pu.x, pu.y, nacc, lane);
        if constexpr (HL) {
          const uint2 pl = s_pvl[w][((bu >> 2) * 4 + sc) * 4 + (bu & 3)];
          pv4_group<D, BITS>(vt, u, pl.x, pl.y, nacc, lane);
        }
      }
      lds_sync_wave();
    }
    vr0 = load_vres(par ^ 1, 0, plan0.nblk);
  }

  // ---- merge the waves and write the chunk partial
  {
    float d = den + row_ror<4>(den);
    d = d + row_ror<8>(d);
    den = pair32_sum(pair16_sum(d));  // lanes with query sc hold its total
  }
  if (lane < 4) s_den[w][lane] = den;
  const long cbase = ((long)bk * a.nsplit + a.chunk_base + chunk) * GQ;
  sum4_waves<D, BITS>(reinterpret_cast<float*>(smem), nacc, w, lane, GQ, a.num + cbase * D);
  if ((int)threadIdx.x < GQ) {
    const int qq = threadIdx.x;
    a.den[cbase + qq] = ((s_den[0][qq] + s_den[1][qq]) + s_den[2][qq]) + s_den[3][qq];
  }
}

int launch_decode_apply4(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.napply_run, A.n_kv_heads, a.B);
  return dispatch_dbs(A.head_dim, A.base_bits, A.scale_mode, [&](auto d, auto bb, auto sm) {
    if (a.k_cap == 1 && a.v_cap == 1)
      hipLaunchKernelGGL((decode_apply4_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value, true>),
                         grid, dim3(256), 0, s, A, a);
    else
      hipLaunchKernelGGL((decode_apply4_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value, false>),
                         grid, dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_apply4");
    return CAREKV_OK;
  });
}

}  // namespace carekv
