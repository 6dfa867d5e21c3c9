// Streaming pass of the CARE-KV decode: one work-group per (split of pages,
// kv head, sequence), 4 waves, one 16-token page per wave iteration.
//
// Per page (lane l: m = l % 16, j = l / 16):
//   * K and V codes of token m, dims [j*D/4, (j+1)*D/4) are dequantised
//     exactly, half(code * scale) (quantizer.py:67-82; int8 scale codes read
//     back as half(code * master), cache.py:713-718), two codes at a time.
//   * S = K_hat q for all query heads of the GQA group on MFMA 16x16x32 f16
//     (rows: tokens, columns: query heads); online softmax in fp32 on the
//     base-2 logits s * log2(e) / sqrt(D).
//   * O += P V_hat on MFMA 16x16x16 f16, V_hat transposed through LDS.
//   * With correction on, the page record: the running max m_ref, for every
//     stored K slot the moments sum dS^2 e^k (k = 2, 3, 4) of
//     e = 2^(x - m_ref), dS = q_cg . R_K / sqrt(D), and for every stored V
//     block the mass sum e.  Those give the query-aware K score
//     (attention.py:167-184) and the V score (attention.py:788-790) once the
//     global softmax statistics are known (select kernel).
// The next page's codes, scales and metadata are loaded while the current
// page is processed.
//
// PF (prefill rows, BITS = 16): the entry's rows come from the prompt's
// dense fp16 K_hat / V_hat; tokens past the entry's row are masked; the
// reference max is the row's log-sum-exp, fixed for every page, so that
// e_t = half(2^(x_t - lse2)) is the reference's fp16 attention weight
// (layer.py:964) and the moments and masses are taken over it.
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

template <int D, int BITS, int SM, bool PF = false>
// 4 waves per SIMD (2 for the fp16 base, whose rows take twice the
// registers): the register budget is capped at 128 (256) VGPRs.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BITS == 16 ? 2 : 4, 8)))
void decode_stream_kernel(carekv_arena A, DecodeArgs a) {
  using G = PageGeom<D, BITS>;
  constexpr int NT = G::NT, NCG = G::NCG, CH = G::CH;
  constexpr int VT_WORDS = kPage * G::VROW;          // one wave's V tile
  constexpr int MERGE_BYTES = 4 * 16 * (D / 2) * 4;  // [4 waves][16 queries][D/2] fp32, two rounds
  constexpr int TILE_BYTES = 4 * VT_WORDS * 4;
  constexpr int LDS_BYTES = MERGE_BYTES > TILE_BYTES ? MERGE_BYTES : TILE_BYTES;
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ __align__(16) _Float16 sq[16 * D];
  __shared__ __align__(16) _Float16 sqr[16 * D];
  __shared__ float s_m[4][16], s_l[4][16];

  // prefill rows: the latest (longest) rows first
  const int split = blockIdx.x, kvh = blockIdx.y, b = a.pf ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  // the call's status word starts clear; the select kernel (a later launch) sets it
  if (((a.split_base + split) | kvh | b) == 0 && threadIdx.x == 0) *a.err_flag = 0;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const EntryRow er = entry_row(A, a, b);
  const int seq = er.seq, np = er.np;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  RowRes rr;
  if constexpr (PF) {
    static_assert(BITS == 16, "prefill rows are fp16");
    const long off = (long)kvh * a.pf_T * D;  // rows past the prompt read as 0
    const uint32_t bytes = (uint32_t)a.pf_T * D * 2;
    rr.kc = make_rsrc(a.pf_k + off, bytes);
    rr.vc = make_rsrc(a.pf_v + off, bytes);
    rr.ks = make_rsrc(nullptr, 0u);
    rr.vs = make_rsrc(nullptr, 0u);
  } else {
    rr = row_resources<D, BITS, SM>(A, pg_base);
  }
  const bool corr = a.correction != 0;
  const float sm_log2 = a.sm_log2;
  const long rq = (long)a.Pmax * a.F;  // record stride between query heads

  if constexpr (PF) {
    stage_q_by<D>(sq, sqr, [&](int n) {
      const PfCol x = pf_col(a, b, kvh, n);
      return x.ok ? a.q + pf_row_off(a, x) * D : (const uint16_t*)nullptr;
    });
  } else {
    stage_q<D>(sq, sqr, a.q + ((long)b * a.Hq + kvh * GQ) * D, GQ);
  }
  __syncthreads();
  half8_t qB[G::NS];
  load_q_operand<D, BITS>(qB, sq, ln, lj);

  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * VT_WORDS;
  float m_run = -INFINITY, l_run = 0.f;
  float x_max = -INFINITY;  // prefill rows with the sketch proxy: the column's largest logit
  int ntok_l = 0;  // prefill rows: tokens the lane's query column sees
  if constexpr (PF) {  // lane column ln (padding columns hold zero queries)
    const PfCol x = pf_col(a, b, kvh, ln);
    m_run = x.ok ? a.pf_lse[(long)x.head * a.pf_T + x.row] * 1.4426950408889634f : 0.f;
    ntok_l = x.ok ? x.row + 1 : 0;
  }
  float4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = float4_t{0.f, 0.f, 0.f, 0.f};

  int p_lo, p_hi;
  launch_pages(A, a, seq, np, p_lo, p_hi);
  const int p_begin = p_lo + split * a.SP, p_end = min(p_begin + a.SP, p_hi);

  PageRegs<D, BITS> nx;
  int nmv = 0;  // next page's metadata, one field per lane
  int p = p_begin + w;
  if (p < p_end) {
    load_page_regs<D, BITS, SM>(nx, rr, p, ln, lj);
    nmv = meta_lanes_load<NCG>(A, pg_base + p, lane);
  }
  for (; p < p_end; p += 4) {
    const PageRegs<D, BITS> cur = nx;
    const PageMeta<NCG> cm = meta_from_lanes<NCG>(nmv, A);
    if (p + 4 < p_end) {
      load_page_regs<D, BITS, SM>(nx, rr, p + 4, ln, lj);
      nmv = meta_lanes_load<NCG>(A, pg_base + p + 4, lane);
    }
    const float ckm = h2f((uint16_t)cm.kmaster), cvm = h2f((uint16_t)cm.vmaster);
    const int nv = PF ? min(cm.nv, er.ntok - p * kPage) : cm.nv;
    if (nv <= 0) continue;
    // K residual rows of the stored slots, issued before the page math
    uint32_t krow[NCG];
    if (corr && cm.meta && !a.proxy) {
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        krow[cg] = 0u;
        if (cm.ksl[cg] >= 0) {
          const long so = (long)seq * A.n_slots + cm.ksl[cg];
          const __amdgpu_buffer_rsrc_t r = make_rsrc(A.k_res + so * G::KSB, G::KSB);
          krow[cg] = __builtin_amdgcn_raw_buffer_load_b32(r, ln * 16 + lj * 4, 0, 0);
        }
      }
    }
    // ---- S = K_hat q
    const _Float16 ks = lane_scale<SM>(cur.ksc, ckm), vs = lane_scale<SM>(cur.vsc, cvm);
    const float4_t sacc = page_scores<D, BITS>(cur.kw, ks, qB);
    // ---- V_hat pairs to LDS while the softmax runs
    {
      half2_t vp[CH / 2];
      dequant_pairs<BITS, CH, BITS>(cur.vw, vs, vp);
      vtile_write<D, BITS>(vt, vp, ln, lj);
    }
    // lane (n = query, j): sacc[i] = S[token 4j+i][query n]
    float x[4];
    if constexpr (PF) {  // the causal limit of the lane's column
      const int nvl = min(nv, ntok_l - p * kPage);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = (4 * lj + i < nvl) ? sacc[i] * sm_log2 : -INFINITY;
    } else if (nv >= kPage) {
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = sacc[i] * sm_log2;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = (4 * lj + i < nv) ? sacc[i] * sm_log2 : -INFINITY;
    }
    if (a.xbuf && corr && ln < GQ)  // logits for the proxy's margins / the entropy
      *reinterpret_cast<float4*>(a.xbuf + (((long)bk * GQ + ln) * a.Pmax + p) * 16 + 4 * lj) =
          make_float4(x[0], x[1], x[2], x[3]);
    if constexpr (PF) x_max = fmaxf(x_max, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
    float m_new, f_old;
    if constexpr (PF) {
      m_new = m_run;
      f_old = 1.f;
    } else {
      const float mx = col_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
      m_new = fmaxf(m_run, mx);  // finite: token 0 of a page is always valid
      f_old = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first page
      m_run = m_new;
    }
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
      if constexpr (PF) e[i] = (float)(_Float16)e[i];
    }
    l_run = l_run * f_old + col_sum((e[0] + e[1]) + (e[2] + e[3]));
    if (__builtin_expect(__any(f_old != 1.f), 0)) {
      // rows of oacc are queries 4j+i: their factors live in lanes 4j+i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float fi = __shfl(f_old, 4 * lj + i, 64);
#pragma unroll
        for (int t = 0; t < NT; ++t) oacc[t][i] *= fi;
      }
    }
    half4_t ap;
    ap[0] = (_Float16)e[0]; ap[1] = (_Float16)e[1]; ap[2] = (_Float16)e[2]; ap[3] = (_Float16)e[3];
    // ---- O += P V_hat
    lds_sync_wave();
    pv_accumulate<D, BITS>(vt, ap, oacc, ln, lj);

    if (corr && cm.meta) {
      // ---- page record (layout in decode_common.h)
      float* rec = a.rec + ((long)bk * GQ * a.Pmax + p) * a.F + ln * rq;
      // t*: the page's first token of largest e for the lane's query (istar:
      // its index among the lane's 4 tokens, out of range in the other lanes)
      const float emax = col_max(fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3])));
      int fi = 4;
#pragma unroll
      for (int i = 3; i >= 0; --i)
        if (e[i] == emax) fi = i;
      const float tstar = -col_max(-(fi < 4 ? (float)(4 * lj + fi) : 16.f));
      const int istar = (int)tstar - 4 * lj;
      if (lj == 0 && ln < GQ) {
        rec[0] = m_new;
        rec[1 + 4 * a.k_cap] = emax;
      }
      if (ln < GQ)
        *reinterpret_cast<uint2*>(a.ebuf + (((long)bk * GQ + ln) * a.Pmax + p) * 16 + 4 * lj) =
            make_uint2(h2bits(half2_t{ap[0], ap[1]}), h2bits(half2_t{ap[2], ap[3]}));
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        const int slot = cm.ksl[cg];
        if (slot < 0) continue;
        if (rk >= a.k_cap) break;  // flagged by the select kernel
        if (a.proxy) { ++rk; continue; }  // the sketch proxy scores K slots without the moments
        const long so = (long)seq * A.n_slots + slot;
        const float4_t racc = kslot_dot_w(krow[cg], sqr, D, cg, ln, lj);
        // moments of u = racc * e over the tokens other than t* (dS = racc
        // * f scales them by f^2): M2 = sum u^2, M3 = sum u^2 e, M4 = sum
        // (u e)^2; D* = racc_t*^2
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
        // reduce over the 4 token groups j: group j ends with the j-th of
        // M2, M3, M4, D*
        const float mj = moments_reduce4(M2, M3, M4, Ds);
        if (ln < GQ) {
          const float f = h2f(A.k_res_scale[so]) * a.inv_sqrt_d;
          rec[1 + 4 * rk + lj] = mj * (f * f);
        }
        ++rk;
      }
      int rv = 0, my_rank = -1;
#pragma unroll
      for (int vb = 0; vb < kVtb; ++vb) {
        if (cm.vsl[vb] < 0) continue;
        if (vb == lj) my_rank = rv;
        ++rv;
      }
      if (my_rank >= 0 && my_rank < a.v_cap && ln < GQ) rec[2 + 4 * a.k_cap + my_rank] = (e[0] + e[1]) + (e[2] + e[3]);
    }
    lds_sync_wave();
  }

  if constexpr (PF) {
    // s_top of the router's margins (residual_router.py:126): the softmax here
    // runs against the row's fixed log-sum-exp, so the maximum logit of each
    // column is kept on the side, per wave
    x_max = col_max(x_max);
    if (a.xmax && lj == 0) a.xmax[(((long)bk * a.nsplit + split) * 4 + w) * 16 + ln] = x_max;
  }
  // ---- merge the 4 waves' (m, l, O) and write the split partial, half
  // of the dims per round; V slot 16t + n (tile t, column n) maps back to dim
  // chunk*CH + slot_code[slot % CH].
  merge_waves<D, BITS>(reinterpret_cast<float*>(smem), s_m, s_l, m_run, l_run, oacc, w, ln, lj, GQ,
                       a.po + ((long)bk * a.nsplit + a.split_base + split) * 16 * D,
                       a.pml + ((long)bk * a.nsplit + a.split_base + split) * 16 * 2);
}

int launch_decode_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit_run, A.n_kv_heads, a.B);
  if (a.pf) {
    // one split (the host's choice when the rows take the work-group-per-8-entries pass)
    if (a.pf_rows) return launch_pf_rows_stream(A, a, s);
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, A, a);
      CAREKV_CHECK_LAUNCH("decode_stream (prefill rows)");
      return CAREKV_OK;
    };
    return A.head_dim == 64 ? go(decode_stream_kernel<64, 16, 0, true>) : go(decode_stream_kernel<128, 16, 0, true>);
  }
  if (A.base_bits != 16 && a.GQ <= 4 && a.SP % 16 == 0)
    return launch_decode_stream4(A, a, s);  // 4-page windows, 4x4x4 MFMA
  return dispatch_dbs16(A.head_dim, A.base_bits, A.scale_mode, [&](auto d, auto bb, auto sm) {
    hipLaunchKernelGGL((decode_stream_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value>), grid,
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_stream");
    return CAREKV_OK;
  });
}

}  // namespace carekv
