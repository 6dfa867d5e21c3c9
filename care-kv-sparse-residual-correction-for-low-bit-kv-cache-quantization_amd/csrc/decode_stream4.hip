// Streaming pass of the CARE-KV decode for GQA groups of at most 4 query
// heads (same inputs and outputs as decode_stream.hip): one work-group per
// (split of pages, kv head, sequence), 4 waves, a window of 4 consecutive
// pages (64 tokens) per wave iteration.
//
// K side, one token row per lane (lane l = token l % 16 of page l / 16):
//   * the lane dequantises its whole K row exactly, half(code * scale)
//     (quantizer.py:67-82, cache.py:713-718), two codes at a time;
//   * S = K_hat q on v_mfma_f32_4x4x4_16b_f16, 16 blocks: block b = tokens
//     4b..4b+3 (rows), column c = query head c; lane 4b + c receives
//     S[4b..4b+3][c], so every lane holds logits of a real (token, query)
//     pair and the softmax and K-slot moments run without padding columns;
//   * online softmax over the window on base-2 logits in fp32;
//   * for every stored K slot of the window's pages, dS = q_cg . R_K on the
//     same MFMA layout and the moments sum dS^2 e^k (k = 2, 3, 4).
// V side, per page (lane l: token l % 16, dims [(l/16) D/4, ...)):
//   V_hat through the padded LDS tile, O^T += V_hat^T P^T on 4x4x4 blocks
//   (A from the tile by the transpose load, P moved from the S layout by
//   ds_bpermute), so the accumulator holds only the 4 query heads.
// The page records and split partials are those of decode_stream.hip, with
// m_ref the running max at the window.
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

// One window's share of a lane: the K side (K rows and scales; reloaded for
// the next window once the window's PV is done, so the records and the next
// window's top cover the latency) and the V side (fetched a whole window
// ahead).  The register cap of 4 waves per SIMD holds with both in flight.
template <int D, int BITS, int SM>
struct WinK {
  static constexpr int RB = row_bytes(D, BITS), NWR = RB / 4, NCG = D / 32;
  static constexpr int KSW = SM == 1 ? (NCG + 3) / 4 : (2 * NCG + 3) / 4;  // K scale words of a row
  uint32_t kw[NWR];
  uint32_t ksc[KSW];
  int meta;  // field (lane % 16) of page (lane / 16)
};
template <int D, int BITS, int SM>
struct WinV {
  static constexpr int NWC = PageGeom<D, BITS>::NWC;
  static constexpr int VSW = SM == 1 ? 1 : 2;  // V scale words (4 pages)
  uint32_t vw[4][NWC];
  uint32_t vsc[VSW];
};

template <int D, int BITS, int SM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void decode_stream4_kernel(carekv_arena A, DecodeArgs a) {
  using G = PageGeom<D, BITS>;
  using WK = WinK<D, BITS, SM>;
  using WV = WinV<D, BITS, SM>;
  using PF = Pairs<BITS, D, BITS>;  // pair schedule of a whole row
  using PR = Pairs<4, 32, 4>;       // pair schedule of a K residual row
  constexpr int NCG = G::NCG, CH = G::CH, RB = G::RB, CHB = G::CHB;
  constexpr int NS4 = D / 4;        // 4x4x4 steps over the head dim
  constexpr int VT_WORDS = kPage * G::VROW;
  constexpr int MERGE_BYTES = 4 * 4 * D * 4;  // [wave][query][D] fp32
  constexpr int TILE_BYTES = 4 * VT_WORDS * 4;
  constexpr int LDS_BYTES = MERGE_BYTES > TILE_BYTES ? MERGE_BYTES : TILE_BYTES;
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ __align__(16) _Float16 sq4[NS4 * 16];       // [step][query][4]: q in the row pair order
  __shared__ __align__(16) _Float16 sqr4[NCG * 8 * 16];  // [cg][step][query][4]: q in the residual order
  __shared__ float s_m[4][4], s_l[4][4];
  __shared__ __align__(16) uint2 s_pw[4][64];            // per wave: [page][query][token group] weights

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const int seq_raw = a.seq_slot[b], np_raw = a.n_pages[b];
  const bool row_ok = seq_raw >= 0 && seq_raw < A.n_seq && np_raw >= 0 && np_raw <= a.Pmax;
  const int seq = row_ok ? seq_raw : 0, np = row_ok ? np_raw : 0;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;  // V side: token ln, chunk lj; K side: token ln of page lj
  const int sc = lane & 3, sbk = ln >> 2;    // S layout: query sc, tokens 4*sbk.. of page lj
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const int p_begin = split * a.SP, p_end = min(p_begin + a.SP, np);
  // code and scale loads past page p_end read out of range of the resources
  // (0, no memory access), so every prefetch is issued unconditionally and
  // the in-order load counter never waits across a branch
  const RowRes rr = row_resources<D, BITS, SM>(A, pg_base, p_end);
  const bool corr = a.correction != 0;
  const float sm_log2 = a.sm_log2;
  const long rq = (long)a.Pmax * a.F;  // record stride between query heads
  float* rec_q = a.rec + ((long)bk * GQ + sc) * rq;  // this lane's query (valid when sc < GQ)

  {  // q in the MFMA orders
    const uint16_t* qg = a.q + ((long)b * a.Hq + kvh * GQ) * D;
    for (int i = threadIdx.x; i < NS4 * 16; i += 256) {
      const int s = i >> 4, c = (i >> 2) & 3, e = i & 3;
      sq4[i] = c < GQ ? bits2half(qg[c * D + PF::T.slot_code[4 * s + e]]) : (_Float16)0.f;
    }
    for (int i = threadIdx.x; i < NCG * 128; i += 256) {
      const int cg = i >> 7, s = (i >> 4) & 7, c = (i >> 2) & 3, e = i & 3;
      sqr4[i] = c < GQ ? bits2half(qg[c * D + cg * 32 + PR::T.slot_code[4 * s + e]]) : (_Float16)0.f;
    }
  }
  __syncthreads();

  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * VT_WORDS;
  float m_run = -INFINITY, l_run = 0.f;
  float4_t oacc[D / 64];  // O[query sc][slots 64h + 4(lane/4) .. +3]
#pragma unroll
  for (int h = 0; h < D / 64; ++h) oacc[h] = float4_t{0.f, 0.f, 0.f, 0.f};

  // K rows and scales of the window, page metadata (one field per lane),
  // V codes and scales one window ahead
  WK kx;
  auto load_k = [&](int q0) {
    const uint32_t krow = (uint32_t)((q0 + lj) * kPage + ln);
    buf_load_row<RB>(kx.kw, rr.kc, krow * RB);
    if constexpr (SM == 1) {
      if constexpr (NCG == 4) kx.ksc[0] = __builtin_amdgcn_raw_buffer_load_b32(rr.ks, krow * NCG, 0, 0);
      else kx.ksc[0] = __builtin_amdgcn_raw_buffer_load_b16(rr.ks, krow * NCG, 0, 0);
    } else {
      if constexpr (NCG == 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rr.ks, krow * NCG * 2, 0, 0);
        kx.ksc[0] = v[0]; kx.ksc[1] = v[1];
      } else {
        kx.ksc[0] = __builtin_amdgcn_raw_buffer_load_b32(rr.ks, krow * NCG * 2, 0, 0);
      }
    }
  };
  auto load_meta = [&](int q0) {
    const int pk = q0 + lj;
    return meta_field_any<NCG, SM>(A, pg_base, pk, pk < p_end, ln);
  };
  auto load_v = [&](WV& v, int q0) {
    const int gi = (lj * CH) / 32;
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      const uint32_t vrow = (uint32_t)((q0 + pi) * kPage + ln);
      buf_load<CHB>(v.vw[pi], rr.vc, vrow * RB + lj * CHB);
    }
    if constexpr (SM == 1) {
      uint32_t sv = 0;
#pragma unroll
      for (int pi = 0; pi < 4; ++pi)
        sv |= (__builtin_amdgcn_raw_buffer_load_b8(rr.vs, (uint32_t)((q0 + pi) * kPage + ln) * NCG + gi, 0, 0) &
               0xffu) << (8 * pi);
      v.vsc[0] = sv;
    } else {
      uint32_t s0 = 0, s1 = 0;
#pragma unroll
      for (int pi = 0; pi < 4; ++pi) {
        const uint32_t h =
            __builtin_amdgcn_raw_buffer_load_b16(rr.vs, ((uint32_t)((q0 + pi) * kPage + ln) * NCG + gi) * 2, 0, 0) &
            0xffffu;
        if (pi < 2) s0 |= h << (16 * pi);
        else s1 |= h << (16 * (pi - 2));
      }
      v.vsc[0] = s0; v.vsc[1] = s1;
    }
  };

  int p0 = p_begin + 4 * w;
  int meta_nx = 0;
  WV vn;
  if (p0 < p_end) {
    load_k(p0);
    meta_nx = load_meta(p0);
    load_v(vn, p0);
  }
  for (; p0 < p_end; p0 += 16) {
    const int cmeta = meta_nx;  // page metadata of this window
    const WV cv = vn;           // V of this window
    load_v(vn, p0 + 16);
    int nvp[4];
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) nvp[pi] = __builtin_amdgcn_readlane(cmeta, 16 * pi);
    const int my_nv = __shfl(cmeta, lane & 48, 64);        // valid tokens of this lane's page
    const int my_meta = __shfl(cmeta, (lane & 48) + 1, 64);

    // ---- S = K_hat q on 4x4x4 blocks
    _Float16 ksg[NCG];
    {
      const float km = SM == 1 ? h2f((uint16_t)__shfl(cmeta, (lane & 48) + 10, 64)) : 0.f;
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        if constexpr (SM == 1) ksg[g] = (_Float16)((float)(int8_t)(kx.ksc[0] >> (8 * g)) * km);
        else ksg[g] = bits2half((uint16_t)(kx.ksc[g >> 1] >> (16 * (g & 1))));
      }
    }
    float4_t sa0 = {0.f, 0.f, 0.f, 0.f}, sa1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS4; ++s) {
      const int g = PF::T.a[2 * s] / 32;
      const half2_t ss = {ksg[g], ksg[g]};
      const half2_t c0 = code_pair<BITS, D, BITS>(kx.kw, 2 * s) * ss;
      const half2_t c1 = code_pair<BITS, D, BITS>(kx.kw, 2 * s + 1) * ss;
      const half4_t ak = {c0[0], c0[1], c1[0], c1[1]};
      const half4_t bq = *reinterpret_cast<const half4_t*>(sq4 + (s * 4 + sc) * 4);
      if (s & 1) sa1 = mfma4x4(ak, bq, sa1);
      else sa0 = mfma4x4(ak, bq, sa0);
    }

    // ---- online softmax over the window (lane: tokens 4*sbk+i of page lj, query sc)
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (4 * sbk + i < my_nv) ? (sa0[i] + sa1[i]) * sm_log2 : -INFINITY;
    if (a.xbuf && corr && sc < GQ && my_nv > 0)  // logits for the proxy's margins / the entropy
      *reinterpret_cast<float4*>(a.xbuf + (((long)bk * GQ + sc) * a.Pmax + p0 + lj) * 16 + 4 * sbk) =
          make_float4(x[0], x[1], x[2], x[3]);
    const float mx = pair32_max(pair16_max(row4_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])))));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // a window with no valid token so far
    const float f_old = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
    l_run = l_run * f_old + pair32_sum(pair16_sum(row4_sum((e[0] + e[1]) + (e[2] + e[3]))));
    if (__builtin_expect(__any(f_old != 1.f), 0)) {
#pragma unroll
      for (int h = 0; h < D / 64; ++h) oacc[h] *= f_old;  // the lane's own query
    }
    const uint32_t e01 = pack_h2(e[0], e[1]), e23 = pack_h2(e[2], e[3]);
    pw_store_strided(s_pw[w], e01, e23, lane);

    // ---- O += P V_hat, page by page
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      if (nvp[pi] <= 0) continue;
      float vm = 0.f;
      if constexpr (SM == 1) vm = h2f((uint16_t)__builtin_amdgcn_readlane(cmeta, 16 * pi + 11));
      _Float16 vs;
      if constexpr (SM == 1) vs = (_Float16)((float)(int8_t)(cv.vsc[0] >> (8 * pi)) * vm);
      else vs = bits2half((uint16_t)(cv.vsc[pi >> 1] >> (16 * (pi & 1))));
      half2_t vp[CH / 2];
      dequant_pairs<BITS, CH, BITS>(cv.vw[pi], vs, vp);
      vtile_write<D, BITS>(vt, vp, ln, lj);
      lds_sync_wave();
      uint2 pg[4];  // P[query sc][tokens g, g+4, g+8, g+12] of page pi
      pw_load(s_pw[w], pi, sc, pg);
#pragma unroll
      for (int g = 0; g < 4; ++g) pv4_group<D, BITS>(vt, g, pg[g].x, pg[g].y, oacc, lane);
      lds_sync_wave();
    }

    load_k(p0 + 16);  // the next window's K rows and metadata
    meta_nx = load_meta(p0 + 16);
    if (!corr) continue;
    // ---- page records: m_ref, K-slot moments, V-block masses (this lane:
    // page lj, query sc; the lanes with sbk == 0 write)
    const int my_page = p0 + lj;
    const bool rec_lane = sc < GQ && my_meta != 0 && my_nv > 0;
    float* rec = rec_q + (long)my_page * a.F;
    if (rec_lane && sbk == 0) rec[0] = m_new;
    if (rec_lane)
      *reinterpret_cast<uint2*>(a.ebuf + (((long)bk * GQ + sc) * a.Pmax + my_page) * 16 + 4 * sbk) = make_uint2(e01, e23);
    int kslot[NCG];
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      const int s = __shfl(cmeta, (lane & 48) + 2 + cg, 64);
      kslot[cg] = (my_meta != 0 && s >= 0 && s < A.n_slots) ? s : -1;
    }
    int nks = 0;
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) nks += kslot[cg] >= 0;
    if (nks > a.k_cap && sbk == 0 && sc == 0) *a.err_flag = 1;
    const int n_mom = a.proxy ? 0 : a.k_cap;  // the sketch proxy scores K slots without the moments
    for (int r = 0; r < n_mom; ++r) {
      int cgr = -1, slotr = -1, cnt = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        if (kslot[cg] < 0) continue;
        if (cnt == r) { cgr = cg; slotr = kslot[cg]; }
        ++cnt;
      }
      const bool has = cgr >= 0;
      if (!__any(has)) break;
      uint32_t rw[4] = {0u, 0u, 0u, 0u};
      if (has) {
        const uint4 v = *reinterpret_cast<const uint4*>(A.k_res + ((long)seq * A.n_slots + slotr) * G::KSB + ln * 16);
        rw[0] = v.x; rw[1] = v.y; rw[2] = v.z; rw[3] = v.w;
      }
      const int cgq = has ? cgr : 0;
      float4_t racc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const half2_t c0 = code_pair<4, 32, 4>(rw, 2 * s);
        const half2_t c1 = code_pair<4, 32, 4>(rw, 2 * s + 1);
        const half4_t ar = {c0[0], c0[1], c1[0], c1[1]};
        const half4_t bq = *reinterpret_cast<const half4_t*>(sqr4 + ((cgq * 8 + s) * 4 + sc) * 4);
        racc = mfma4x4(ar, bq, racc);
      }
      // moments of u = racc * e (dS = racc * f scales them by f^2)
      float M2 = 0.f, M3 = 0.f, M4 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = racc[i] * e[i];
        const float ue = u * e[i];
        M2 = fmaf(u, u, M2);
        M3 = fmaf(ue, u, M3);
        M4 = fmaf(ue, ue, M4);
      }
      M2 = row4_sum(M2); M3 = row4_sum(M3); M4 = row4_sum(M4);
      if (has && rec_lane && sbk == 0) {
        const float f = h2f(A.k_res_scale[(long)seq * A.n_slots + slotr]) * a.inv_sqrt_d;
        const float f2 = f * f;
        rec[1 + 3 * r] = M2 * f2; rec[2 + 3 * r] = M3 * f2; rec[3 + 3 * r] = M4 * f2;
      }
    }
    // V block sbk of page lj: its stored-slot rank and mass
    int vrank = -1, rv = 0;
#pragma unroll
    for (int vb = 0; vb < kVtb; ++vb) {
      const int s = __shfl(cmeta, (lane & 48) + 6 + vb, 64);
      if (s < 0 || s >= A.n_slots) continue;
      if (vb == sbk) vrank = rv;
      ++rv;
    }
    if (rec_lane && vrank >= 0) {
      if (vrank < a.v_cap) rec[1 + 3 * a.k_cap + vrank] = (e[0] + e[1]) + (e[2] + e[3]);
      else *a.err_flag = 1;
    }
  }

  merge4_waves<D, BITS>(reinterpret_cast<float*>(smem), s_m, s_l, m_run, l_run, oacc, w, lane, GQ,
                       a.po + ((long)bk * a.nsplit + split) * 16 * D,
                       a.pml + ((long)bk * a.nsplit + split) * 16 * 2);
}

int launch_decode_stream4(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, A.n_kv_heads, a.B);
  return dispatch_dbs(A.head_dim, A.base_bits, A.scale_mode, [&](auto d, auto bb, auto sm) {
    hipLaunchKernelGGL((decode_stream4_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value>), grid,
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_stream4");
    return CAREKV_OK;
  });
}

}  // namespace carekv
