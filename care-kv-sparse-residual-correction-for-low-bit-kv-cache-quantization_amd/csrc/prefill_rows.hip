// Streaming pass of the prefill correction (carekv_prefill_correct) over
// blocks of prompt rows, flash style: the records, stored weights and base
// output that decode_stream_kernel<D, 16, 0, true> forms entry by entry,
// formed for 4 entries at once from K_hat / V_hat tiles staged in LDS.
//
// An entry packs R = 16 / G0 consecutive prompt rows of one kv head into 16
// query columns (column c = row c / G0, head c % G0; PfCol).  The
// entry-per-work-group pass reads every visible page once per entry, i.e.
// once per R rows; here a work-group takes 4 QB consecutive entries of a
// kv head (QB per wave, one per 16-column MFMA sub-block), so each 32-token
// tile (two pages) is read once for 4 QB R rows:
//   * S = K_hat q on v_mfma_f32_16x16x32_f16 in the generic kernel's
//     reduction order (lane (column n, group j): tokens 4j..4j+3 of the
//     page; step s over the dims j D/4 + 8s ..), so S, e, the records and
//     the stored weights are the generic kernel's bits;
//   * e_t = half(2^(x_t - lse2)) against the row's fixed log-sum-exp
//     (layer.py:964), masked past the row and past the page's valid rows;
//   * per (column, page) the generic kernel's record: m_ref, t* and e*, the
//     K slots' moments (dS on the same MFMA from the residual rows), the V
//     blocks' masses, and the fp16 weights (ebuf);
//   * O += e V_hat on the same tile (transpose load), and L = sum e, as the
//     entry's partial of the work-group's split.
// The grid's third dimension splits the pages (SP a split): a row's work
// grows with its index, and with all of a prompt's entries resident at once
// the longest rows' chains of tiles would otherwise run alone at the end.
// Every split's partial carries the same fixed maximum lse2, so the merges
// add the partials with weight exp2(0) = 1: the splits change only the fp32
// order of the O and L sums.  A split past an entry's last page writes no
// partial, and the select and combine kernels read none (splits_read).
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

template <int D, int QB>
__global__ __launch_bounds__(256, 2) void pf_rows_stream_kernel(carekv_arena A, DecodeArgs a) {
  using PK = Pairs<4, 8, 4>;          // K residual pair order inside 8-dim blocks
  constexpr int KT = 32;              // tokens per tile (two pages)
  constexpr int CH = D / 4;           // dims of a lane group's chunk
  constexpr int NS = D / 32;          // 16x16x32 steps of S
  constexpr int NCG = D / 32;
  constexpr int DT = D / 16;          // 16-dim output tiles
  constexpr int KRS = 2 * D + 16;     // K tile row stride, bytes
  constexpr int VRS = 2 * D + 32;     // V tile row stride, bytes
  constexpr int KBUF = KT * KRS, VBUF = KT * VRS, BUF = KBUF + VBUF;
  constexpr int CHR = D / 8;          // 16-byte chunks per row
  constexpr int NCH = 2 * KT * CHR / 256;
  constexpr int EPW = 4 * QB;         // entries per work-group (QB per wave)
  __shared__ __align__(16) char lds[2 * BUF];
  __shared__ __align__(16) _Float16 sqr[EPW * 16 * D];  // q in the residual pair order, [entry][column][D]
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;

  const int kvh = blockIdx.y;
  // the latest (longest) rows first
  const int blk = (int)(gridDim.x - 1 - blockIdx.x);
  const int e0 = blk * EPW;
  if (blk == (int)gridDim.x - 1 && kvh == 0 && threadIdx.x == 0) *a.err_flag = 0;  // the call's status word
  const int GQ = a.GQ, T = a.pf_T;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;
  const int seq = a.pf_seq;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const bool corr = a.correction != 0;
  const float sm_log2 = a.sm_log2;

  // ---- q: the generic kernel's S operands for the wave's two entries, and
  // every entry's q in the residual order for the K slots' dS
  int eb[QB], enp[QB], entok[QB], ntok_l[QB];
  bool eok[QB];
  float lse2[QB];
  half8_t qf[QB][NS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int b = e0 + QB * w + qb;
    eb[qb] = b;
    eok[qb] = b < a.B;
    const EntryRow er = entry_row(A, a, eok[qb] ? b : 0);
    enp[qb] = eok[qb] ? er.np : 0;
    entok[qb] = eok[qb] ? er.ntok : 0;
    const PfCol x = pf_col(a, b, kvh, ln);
    const bool ok = eok[qb] && x.ok;
    lse2[qb] = ok ? a.pf_lse[(long)x.head * T + x.row] * 1.4426950408889634f : 0.f;
    ntok_l[qb] = ok ? x.row + 1 : 0;
    const uint16_t* qp = ok ? a.q + pf_row_off(a, x) * D : nullptr;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (qp) {
        const uint4 v = *reinterpret_cast<const uint4*>(qp + lj * CH + 8 * s);
        __builtin_memcpy(&qf[qb][s], &v, 16);
      } else {
        qf[qb][s] = half8_t{};
      }
    }
  }
  // pages of the work-group: those of its last entry; its split: tiles
  // jt0 .. jt1-1 (SP / 2 tiles a split)
  const int np_wg = entry_row(A, a, min(e0 + EPW, a.B) - 1).np;
  const int nt = (np_wg + 1) / 2;
  const int split = blockIdx.z, tps = a.SP / 2;
  const int jt0 = split * tps, jt1 = min(jt0 + tps, nt);
  if (jt0 >= jt1) return;  // past every entry's pages: no partial (splits_read)
  {  // every entry's q in the residual pair order: thread t fills dims
     // [(t % 4) D/4, ..) of column (t / 4) % 16 of entry t / 64, one column
     // lookup per thread; within each 8-dim block the order is
     // {0, 4, 1, 5, 2, 6, 3, 7}, two byte permutes per pair of output words
    static_assert(EPW * 16 * 4 == 256, "one thread per quarter column");
    static_assert(PK::T.slot_code[0] == 0 && PK::T.slot_code[1] == 4 && PK::T.slot_code[2] == 1 &&
                      PK::T.slot_code[3] == 5 && PK::T.slot_code[4] == 2 && PK::T.slot_code[5] == 6 &&
                      PK::T.slot_code[6] == 3 && PK::T.slot_code[7] == 7,
                  "residual pair order inside an 8-dim block");
    constexpr int DPT = D / 4;
    const int el = threadIdx.x >> 6, n = (threadIdx.x >> 2) & 15, d0 = (threadIdx.x & 3) * DPT;
    const int b = e0 + el;
    const PfCol x = pf_col(a, b, kvh, n);
    const bool ok = b < a.B && x.ok;
    const uint16_t* qr = a.q + (ok ? pf_row_off(a, x) * D : 0) + d0;
    _Float16* dst = sqr + (el * 16 + n) * D + d0;
#pragma unroll
    for (int c = 0; c < DPT; c += 8) {
      const uint4 v = ok ? *reinterpret_cast<const uint4*>(qr + c) : make_uint4(0u, 0u, 0u, 0u);
      // v.x = (h1, h0), v.y = (h3, h2), v.z = (h5, h4), v.w = (h7, h6)
      *reinterpret_cast<uint4*>(dst + c) =
          make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                     __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
    }
  }

  const uint32_t span = (uint32_t)T * D * 2;  // rows past the prompt read as 0
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.pf_k + (long)kvh * T * D, span);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.pf_v + (long)kvh * T * D, span);
  uint32_t stg[NCH][4];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = threadIdx.x + 256 * k;
      const int rc = c % (KT * CHR), row = rc / CHR, col = rc % CHR;
      const uint32_t off = ((uint32_t)(j * KT + row) * D + col * 8) * 2;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(k < NCH / 2 ? rk : rv, off, 0, 0);
      stg[k][0] = v[0]; stg[k][1] = v[1]; stg[k][2] = v[2]; stg[k][3] = v[3];
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = threadIdx.x + 256 * k;
      const int rc = c % (KT * CHR), row = rc / CHR, col = rc % CHR;
      char* dst = lds + buf * BUF + (k < NCH / 2 ? row * KRS : KBUF + row * VRS) + col * 16;
      *reinterpret_cast<uint4*>(dst) = make_uint4(stg[k][0], stg[k][1], stg[k][2], stg[k][3]);
    }
  };
  // Page metadata without a branch on the lane or the page: one dword per
  // lane (lane 0 valid, 2.. k_slot, 6..9 v_slot; the other lanes read valid
  // again, unused) from a per-lane address, and the page's has_meta byte;
  // a page past the work-group's last one reads that last page and is
  // dropped where the metadata is used.  A load under a branch would leave
  // the compiler unable to count the loads in flight, and its wait for the
  // metadata would then also wait for the next tile's K_hat / V_hat loads
  // and for every record store.
  struct MetaRaw { int w, hm; };
  auto load_meta2 = [&](int j, MetaRaw* mv) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const long pg = pg_base + min(2 * j + tt, np_wg - 1);
      const int* src = A.valid + pg;
      if (lane >= 2 && lane < 2 + NCG) src = A.k_slot + pg * NCG + (lane - 2);
      if (lane >= 6 && lane < 6 + kVtb) src = A.v_slot + pg * kVtb + (lane - 6);
      mv[tt].w = *src;
      mv[tt].hm = A.has_meta[pg];
    }
  };
  auto meta_of = [&](const MetaRaw& r, int p) {
    PageMeta<NCG> m{};
    if (p >= np_wg) return m;  // wave-uniform
    m.nv = __builtin_amdgcn_readlane(r.w, 0);
    m.meta = __builtin_amdgcn_readfirstlane(r.hm);
#pragma unroll
    for (int c = 0; c < NCG; ++c) {
      const int sl = __builtin_amdgcn_readlane(r.w, 2 + c);
      m.ksl[c] = sl < A.n_slots ? sl : -1;
    }
#pragma unroll
    for (int v = 0; v < kVtb; ++v) {
      const int sl = __builtin_amdgcn_readlane(r.w, 6 + v);
      m.vsl[v] = sl < A.n_slots ? sl : -1;
    }
    return m;
  };
  // records and stored weights through one buffer resource over the
  // workspace (rec .. xbuf, below 4 GiB): a lane with nothing to write
  // stores past its end, which the hardware drops, so no store sits behind
  // a lane branch either
  const __amdgpu_buffer_rsrc_t rs_ws = make_rsrc(a.rec, a.ws_span);
  constexpr uint32_t kDrop = 0xfffffff0u;
  // K residual words (lane: token ln, bytes 4lj..) and raw fp16 scales of
  // the two pages' stored slots; a page without a slot (or without
  // metadata) reads past the end of the resources, i.e. 0 with no memory
  // access, so that the loads are issued by every lane without a branch
  constexpr int KSB = PageGeom<D, 16>::KSB;
  const __amdgpu_buffer_rsrc_t rkr = make_rsrc(A.k_res + (long)seq * A.n_slots * KSB, (uint32_t)A.n_slots * KSB);
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(A.k_res_scale + (long)seq * A.n_slots, (uint32_t)A.n_slots * 2u);
  auto load_kres = [&](const PageMeta<NCG>* m, uint32_t (*kw)[NCG], uint32_t (*ks)[NCG]) {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const bool has = corr && m[tt].meta && m[tt].ksl[cg] >= 0;
        const uint32_t slot = has ? (uint32_t)m[tt].ksl[cg] : (uint32_t)A.n_slots;
        kw[tt][cg] = __builtin_amdgcn_raw_buffer_load_b32(rkr, slot * KSB + ln * 16 + lj * 4, 0, 0);
        ks[tt][cg] = __builtin_amdgcn_raw_buffer_load_b16(rks, slot * 2u, 0, 0);
      }
  };

  float4_t o[QB][DT];
  float lpart[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    lpart[qb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[qb][dt] = float4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Load schedule: the metadata of tile jt + 1 is in flight during tile jt;
  // the K residual words and scales of a tile are issued at its top, ahead
  // of its S products.  (Issuing them a tile ahead measured the same at 25
  // VGPRs more: the pass is bound by its longest chain of tiles, which the
  // splits keep short, not by these loads.)
  MetaRaw mv_nx[2];
  load_tile(jt0);
  store_tile(0);
  load_meta2(jt0, mv_nx);
  __syncthreads();
  if (jt0 + 1 < jt1) load_tile(jt0 + 1);

  for (int jt = jt0; jt < jt1; ++jt) {
    const char* kb = lds + ((jt - jt0) & 1) * BUF;
    const char* vb = kb + KBUF;
    PageMeta<NCG> cm[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) cm[tt] = meta_of(mv_nx[tt], 2 * jt + tt);
    if (jt + 1 < jt1) load_meta2(jt + 1, mv_nx);
    uint32_t krow[2][NCG], ksc[2][NCG];
    load_kres(cm, krow, ksc);

    // ---- S = K_hat q per page and entry, and the page's weights and record
    float ep[2][QB][4];  // [page][entry][token i]
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      half8_t ak[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        *reinterpret_cast<uint4*>(&ak[s]) =
            *reinterpret_cast<const uint4*>(kb + (16 * tt + ln) * KRS + (lj * CH + 8 * s) * 2);
      const int p = 2 * jt + tt;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NS; ++s) sacc = mfma16x32(ak[s], qf[qb][s], sacc);
#pragma unroll
        for (int i = 0; i < 4; ++i) ep[tt][qb][i] = 0.f;
        // the entry's pages; a page with no visible valid row adds nothing
        if (!eok[qb] || p >= enp[qb]) continue;
        const int nv = min(cm[tt].nv, entok[qb] - p * kPage);
        if (nv <= 0) continue;
        const int nvl = min(nv, ntok_l[qb] - p * kPage);  // the causal limit of the lane's column
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = (4 * lj + i < nvl) ? sacc[i] * sm_log2 : -INFINITY;
          e[i] = (float)(_Float16)__builtin_amdgcn_exp2f(x - lse2[qb]);
          ep[tt][qb][i] = e[i];
        }
        lpart[qb] += (e[0] + e[1]) + (e[2] + e[3]);
        if (!(corr && cm[tt].meta)) continue;
        // ---- page record (layout in decode_common.h)
        const int b = eb[qb];
        const long bk = (long)b * A.n_kv_heads + kvh;
        // byte offsets of this lane's record and stored weights (query ln)
        const uint32_t ro = (uint32_t)(((bk * GQ + ln) * a.Pmax + p) * a.F) * 4u;
        const uint32_t eo = a.ws_e_off + (uint32_t)(((bk * GQ + ln) * a.Pmax + p) * 16 + 4 * lj) * 2u;
        const bool qok = ln < GQ;
        const float emax = col_max(fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3])));
        int fi = 4;
#pragma unroll
        for (int i = 3; i >= 0; --i)
          if (e[i] == emax) fi = i;
        const float tstar = -col_max(-(fi < 4 ? (float)(4 * lj + fi) : 16.f));
        const int istar = (int)tstar - 4 * lj;
        typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
        const uint32_t ro0 = (lj == 0 && qok) ? ro : kDrop;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse2[qb]), rs_ws, ro0, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(emax), rs_ws,
                                              ro0 == kDrop ? kDrop : ro0 + (uint32_t)(1 + 4 * a.k_cap) * 4u, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b64(u2_t{pack_h2(e[0], e[1]), pack_h2(e[2], e[3])}, rs_ws,
                                              qok ? eo : kDrop, 0, 0);
        const _Float16* sqe = sqr + (QB * w + qb) * 16 * D;
        int rkk = 0;
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) {
          const int slot = cm[tt].ksl[cg];
          if (slot < 0) continue;
          if (rkk >= a.k_cap) break;  // flagged by the select kernel
          const float4_t racc = kslot_dot_w(krow[tt][cg], sqe, D, cg, ln, lj);
          float M2 = 0.f, M3 = 0.f, M4 = 0.f, Ds = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (i == istar) {
              Ds = racc[i] * racc[i];
              continue;
            }
            const float u = racc[i] * e[i];
            const float ue = u * e[i];
            M2 = fmaf(u, u, M2);
            M3 = fmaf(ue, u, M3);
            M4 = fmaf(ue, ue, M4);
          }
          const float mj = moments_reduce4(M2, M3, M4, Ds);
          {
            const float f = h2f((uint16_t)ksc[tt][cg]) * a.inv_sqrt_d;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(mj * (f * f)), rs_ws,
                                                  qok ? ro + (uint32_t)(1 + 4 * rkk + lj) * 4u : kDrop, 0, 0);
          }
          ++rkk;
        }
        int rvv = 0, my_rank = -1;
#pragma unroll
        for (int vb2 = 0; vb2 < kVtb; ++vb2) {
          if (cm[tt].vsl[vb2] < 0) continue;
          if (vb2 == lj) my_rank = rvv;
          ++rvv;
        }
        __builtin_amdgcn_raw_buffer_store_b32(
            __float_as_uint((e[0] + e[1]) + (e[2] + e[3])), rs_ws,
            (my_rank >= 0 && my_rank < a.v_cap && qok) ? ro + (uint32_t)(2 + 4 * a.k_cap + my_rank) * 4u : kDrop, 0, 0);
      }
    }

    // ---- O += e V_hat over the tile (tokens 4lj + i of each page)
    {
      half8_t bp[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        bp[qb] = half8_t{(_Float16)ep[0][qb][0], (_Float16)ep[0][qb][1], (_Float16)ep[0][qb][2],
                         (_Float16)ep[0][qb][3], (_Float16)ep[1][qb][0], (_Float16)ep[1][qb][1],
                         (_Float16)ep[1][qb][2], (_Float16)ep[1][qb][3]};
      const __attribute__((address_space(3))) char* vrow =
          (const __attribute__((address_space(3))) char*)vb + (4 * lj + (ln >> 2)) * VRS + (ln & 3) * 8;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrow + 32 * dt));
        const short4_t v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrow + 16 * VRS + 32 * dt));
        half8_t av;
        __builtin_memcpy(&av, &v1, 8);
        __builtin_memcpy(reinterpret_cast<char*>(&av) + 8, &v2, 8);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) o[qb][dt] = mfma16x32(av, bp[qb], o[qb][dt]);
      }
    }
    if (jt + 1 < jt1) store_tile((jt + 1 - jt0) & 1);
    if (jt + 2 < jt1) load_tile(jt + 2);
    __syncthreads();
  }

  // ---- the entries' split partials: O unnormalised, (lse2, L); none for
  // an entry whose pages end before the split (splits_read)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = col_sum(lpart[qb]);
    if (!eok[qb] || ln >= GQ || split * a.SP >= enp[qb]) continue;
    const long bk = (long)eb[qb] * A.n_kv_heads + kvh;
    float* po = a.po + ((bk * a.nsplit + split) * 16 + ln) * D + 4 * lj;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4*>(po + 16 * dt) = make_float4(o[qb][dt][0], o[qb][dt][1], o[qb][dt][2], o[qb][dt][3]);
    if (lj == 0) {
      float* pml = a.pml + ((bk * a.nsplit + split) * 16 + ln) * 2;
      pml[0] = lse2[qb];
      pml[1] = lt;
    }
  }
}

int launch_pf_rows_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  if (!a.pf || a.proxy || a.xbuf || a.SP % 2 != 0 || a.nsplit * a.SP < a.pf_pages) {
    set_error("pf_rows_stream: prefill rows with the moments' K score, no logit buffer and splits of whole tiles "
              "covering every page");
    return CAREKV_EINVAL;
  }
  // one entry per wave (two entries per wave, one wave per SIMD, measured
  // 30% slower), one split per grid layer
  const dim3 grid((a.B + 3) / 4, A.n_kv_heads, a.nsplit);
  if (A.head_dim == 64) hipLaunchKernelGGL((pf_rows_stream_kernel<64, 1>), grid, dim3(256), 0, s, A, a);
  else if (A.head_dim == 128) hipLaunchKernelGGL((pf_rows_stream_kernel<128, 1>), grid, dim3(256), 0, s, A, a);
  else {
    set_error("pf_rows_stream: head_dim %d (kernels: 64, 128)", A.head_dim);
    return CAREKV_EINVAL;
  }
  CAREKV_CHECK_LAUNCH("pf_rows_stream");
  return CAREKV_OK;
}

}  // namespace carekv
