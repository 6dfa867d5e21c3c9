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
//   the raw codes (code_pair_sub form, one bitop3 per pair) through the
//   padded LDS tile, O^T += V^T P'^T on 4x4x4 blocks (A from the tile by the
//   transpose load), so the accumulator holds only the 4 query heads.  The
//   V scales ride on the weights, P'[t][G] = half(half(e_t) * s_V[t][G]);
//   the merge undoes the code offset and the subnormal scaling.  The output
//   differs from sum_t a_t half(code * s) by the fp16 rounding of P' and of
//   half(code * s), within the output tolerance; V_hat enters nothing
//   else of this pass.
// The page records and split partials are those of decode_stream.hip, with
// m_ref the running max at the window.
//
// KV (the packed KIVI prefix, carekv_arena::kivi_packed): 2-bit K codes
// against one per-channel scale vector s_c of the (kv head, sequence).
// K_hat = half(code * s_c) = code * s_c exactly for codes -2..1, so
// S = sum_c (q_c s_c) code_c with every product exact: q_c s_c (22
// significant bits, exact in fp32) is split into fp16 hi + lo, both run
// through the MFMA against the exact integer codes, and the two
// accumulators sum to S up to fp32 order.  A power-of-two 2^E per work-group
// keeps the largest |q_c s_c| 2^E near 2^15 so that hi and lo stay normal;
// S is scaled back by 2^-E.  The V pages are those of a 2-bit base with
// fp16 group scales; the V product runs on exact signed fp16 codes (two ops
// per pair) against the weights P' = half(e) s_V, exact in fp32 and carried
// as fp16 hi + lo, and L sums half(e): the base output and its normaliser
// then weigh V_hat exactly as the apply pass does (half(e) V_hat).  The
// KIVI base's K corrections can remove most of the mass (|dO| above |O|,
// 1 + den / L down to a few hundredths), which amplifies any error of the
// base output: the offset-code form of the uniform bases, whose offset
// 2^(b-1) sum(P') cancels against the code sum, loses about 1e-4 there.
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

// One window's share of a lane: the K side (K rows and scales; reloaded for
// the next window as soon as the S step has consumed them, so the softmax,
// the records and the PV step cover the latency) and the V side (fetched a
// whole window ahead).  The register cap of 4 waves per SIMD holds with both
// in flight because the records run before the PV step, so that their
// registers (the weights, the residual rows) are free during it.
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

template <int D, int BITS, int SM, bool KV = false>
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
  __shared__ __align__(16) _Float16 sq4lo[KV ? NS4 * 16 : 4];  // KV: the lo halves of q_c s_c 2^E
  __shared__ float s_red[4];
  __shared__ __align__(16) _Float16 sqr4[NCG * 8 * 16];  // [cg][step][query][4]: q in the residual order
  __shared__ float s_m[4][4], s_l[4][4];
  __shared__ __align__(16) uint16_t s_pw[4][4 * NCG * 64];  // per wave: [page][G][query][16] weights P'
  __shared__ __align__(16) uint16_t s_pwl[KV ? 4 : 1][KV ? 4 * NCG * 64 : 8];  // KV: their lo halves
  __shared__ __align__(16) uint16_t s_vs[4][4 * NCG * 16];  // per wave: [page][G][token] V scales

  // prefill rows: the latest (longest) rows first
  const int split = blockIdx.x, kvh = blockIdx.y, b = a.pf ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  // the call's status word starts clear; the select kernel (a later launch) sets it
  if ((split | kvh | b) == 0 && threadIdx.x == 0) *a.err_flag = 0;
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
  // the packed KIVI prefix stops at the row's n_packed; its launch (range 1)
  // and the uniform bases' (range 0) both start at split slot 0
  int p_hi = np;
  if constexpr (KV) p_hi = min(np, max(A.n_packed[seq], 0));
  const int p_begin = split * a.SP, p_end = min(p_begin + a.SP, p_hi);
  // code and scale loads past page p_end read out of range of the resources
  // (0, no memory access), so every prefetch is issued unconditionally and
  // the in-order load counter never waits across a branch
  const RowRes rr = row_resources<D, BITS, SM>(A, pg_base, p_end);
  const bool corr = a.correction != 0;
  const float sm_log2 = a.sm_log2;
  const int rq = a.Pmax * a.F;  // record stride between query heads
  // records, stored weights and the K residual slots of (sequence, kv head)
  // through buffer resources: SGPR bases, 32-bit lane offsets
  typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
  // one resource over the workspace from the records to the logits (a
  // span the host keeps below 4 GiB) with per-array SGPR offsets
  const __amdgpu_buffer_rsrc_t rs_ws = make_rsrc(a.rec, a.ws_span);
  const uint32_t so_rec = (uint32_t)(bk * GQ * rq) * 4u;
  const uint32_t so_e = a.ws_e_off + (uint32_t)(bk * GQ * a.Pmax) * 32u;
  const uint32_t so_x = a.ws_x_off + (uint32_t)(bk * GQ * a.Pmax) * 64u;
  // lane parts of the record, weight and logit offsets (page lj, tokens
  // 4*sbk.., query sc); the window start p0 goes into the SGPR offset
  const uint32_t vo_rec = (uint32_t)(sc * rq + lj * a.F) * 4u;
  const uint32_t vo_e = (uint32_t)((sc * a.Pmax + lj) * 16 + 4 * sbk) * 2u;
  const uint32_t vo_x = (uint32_t)((sc * a.Pmax + lj) * 16 + 4 * sbk) * 4u;
  const int8_t* kres_row = A.k_res + (long)seq * A.n_slots * G::KSB;  // K residual slots of the sequence
  const uint16_t* kres_sc = A.k_res_scale + (long)seq * A.n_slots;

  float s_back = 1.f;  // KV: 2^-E
  {  // q in the MFMA orders
    const uint16_t* qg = a.q + ((long)b * a.Hq + kvh * GQ) * D;
    if constexpr (KV) {
      const uint16_t* kc = A.kchan + ((long)kvh * A.n_seq + seq) * D;
      float mx = 0.f;
      for (int i = threadIdx.x; i < NS4 * 16; i += 256) {
        const int s = i >> 4, c = (i >> 2) & 3, e = i & 3, ch = PF::T.slot_code[4 * s + e];
        if (c < GQ) mx = fmaxf(mx, fabsf(h2f(qg[c * D + ch]) * h2f(kc[ch])));
      }
      mx = wave_max(mx);
      if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
      __syncthreads();
      mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
      // |q s| 2^E <= 2^15: the exponent of mx read from its bits (mx normal
      // or 0; a non-finite mx keeps E = 0)
      int E = 0;
      if (mx > 0.f && mx < INFINITY) E = min(max(15 - ((int)((__float_as_uint(mx) >> 23) & 0xffu) - 127) - 1, -100), 100);
      const float up = __builtin_ldexpf(1.f, E);
      s_back = __builtin_ldexpf(1.f, -E);
      for (int i = threadIdx.x; i < NS4 * 16; i += 256) {
        const int s = i >> 4, c = (i >> 2) & 3, e = i & 3, ch = PF::T.slot_code[4 * s + e];
        const float v = c < GQ ? h2f(qg[c * D + ch]) * h2f(kc[ch]) * up : 0.f;  // exact in fp32
        const _Float16 hi = (_Float16)v;
        sq4[i] = hi;
        sq4lo[i] = (_Float16)(v - (float)hi);
      }
    } else {
      for (int i = threadIdx.x; i < NS4 * 16; i += 256) {
        const int s = i >> 4, c = (i >> 2) & 3, e = i & 3;
        sq4[i] = c < GQ ? bits2half(qg[c * D + PF::T.slot_code[4 * s + e]]) : (_Float16)0.f;
      }
    }
    for (int i = threadIdx.x; i < NCG * 128; i += 256) {
      const int cg = i >> 7, s = (i >> 4) & 7, c = (i >> 2) & 3, e = i & 3;
      sqr4[i] = c < GQ ? bits2half(qg[c * D + cg * 32 + PR::T.slot_code[4 * s + e]]) : (_Float16)0.f;
    }
  }
  __syncthreads();

  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * VT_WORDS;
  float m_run = -INFINITY, l_run = 0.f;
  float4_t oacc[D / 64];  // O[query sc][slots 64h + 4(lane/4) .. +3] over raw codes
#pragma unroll
  for (int h = 0; h < D / 64; ++h) oacc[h] = float4_t{0.f, 0.f, 0.f, 0.f};
  float wsum[NCG];  // sum of the lane's weights P'[t][G] (its query, its tokens)
#pragma unroll
  for (int g = 0; g < NCG; ++g) wsum[g] = 0.f;
  const half2_t one2 = {(_Float16)1.f, (_Float16)1.f};

  // K rows and scales of the window, page metadata (one field per lane),
  // V codes and scales one window ahead
  WK kx;
  auto load_k = [&](int q0) {
    const uint32_t krow = (uint32_t)((q0 + lj) * kPage + ln);
    buf_load_row<RB>(kx.kw, rr.kc, krow * RB);
    if constexpr (KV) {
      // no K scales: the channel scales ride on q
    } else if constexpr (SM == 1) {
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
    return meta_field_row<NCG, SM>(A, pg_base, pk, pk < p_end, ln);
  };
  auto load_vpage = [&](WV& v, int q0, int pi) {
    const uint32_t vrow = (uint32_t)((q0 + pi) * kPage + ln);
    buf_load<CHB>(v.vw[pi], rr.vc, vrow * RB + lj * CHB);
  };
  auto load_vscale = [&](WV& v, int q0) {
    const int gi = (lj * CH) / 32;
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

  // Load schedule of a window (one register set per buffer): this
  // window's first K residual rows at the top; the next window's K rows and
  // metadata right after the S step has consumed the K registers; the next
  // window's V codes page by page as the PV step consumes them, its V
  // scales once they are in LDS.  The loads complete in issue order, so
  // the records wait for nothing issued after the top, and the next
  // window's S step has the softmax, the records and the PV step of this
  // one to wait through.
  int p0 = p_begin + 4 * w;
  int meta_nx = 0;
  WV cv;
  if (p0 < p_end) {
    load_k(p0);
    meta_nx = load_meta(p0);
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) load_vpage(cv, p0, pi);
    load_vscale(cv, p0);
  }
  const bool mom = corr && !a.proxy && a.k_cap > 0;  // the sketch proxy scores K slots without the moments
  for (; p0 < p_end; p0 += 16) {
    const int cmeta = meta_nx;  // page metadata of this window
    const int my_meta = __shfl(cmeta, (lane & 48) + 1, 64);
    // stored K slots of the lane's page (the metadata lanes' ballots: bit
    // 16*pi + f = field f of page pi names a slot inside the arena) and the
    // first one's residual row
    const int fld = lane & 15;
    const bool in_arena = cmeta >= 0 && cmeta < A.n_slots;
    const uint64_t kbal = __ballot(fld >= 2 && fld < 2 + NCG && in_arena);
    const uint64_t vbal = __ballot(fld >= 6 && fld < 6 + kVtb && in_arena);
    const uint32_t kmask0 = my_meta != 0 ? (uint32_t)(kbal >> (16 * lj + 2)) & ((1u << NCG) - 1u) : 0u;
    uint32_t rw0[4] = {0u, 0u, 0u, 0u};
    uint32_t ksc0 = 0u;
    if (mom) {
      const int cg0 = kmask0 ? (int)__builtin_ctz(kmask0) : 0;
      const int slot0 = __shfl(cmeta, (lane & 48) + 2 + cg0, 64);
      const uint32_t soff0 = kmask0 ? (uint32_t)slot0 : 0u;  // lanes without a slot read slot 0 and drop it
      const uint4 v = ld_off<uint4>(kres_row, soff0 * G::KSB + ln * 16);
      rw0[0] = v.x; rw0[1] = v.y; rw0[2] = v.z; rw0[3] = v.w;
      ksc0 = ld_off<uint16_t>(kres_sc, soff0 * 2u);
    }
    int nvp[4];
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) nvp[pi] = __builtin_amdgcn_readlane(cmeta, 16 * pi);
    const int my_nv = __shfl(cmeta, lane & 48, 64);        // valid tokens of this lane's page

    // ---- V scales of the window to LDS ([page][G][token]); the V-layout
    // lane (token ln, chunk lj) holds those of its token and group
    {
      const int gi = (lj * CH) / 32;
#pragma unroll
      for (int pi = 0; pi < 4; ++pi) {
        _Float16 vs;
        if constexpr (SM == 1) {
          const float vm = h2f((uint16_t)__builtin_amdgcn_readlane(cmeta, 16 * pi + 11));
          vs = (_Float16)((float)(int8_t)(cv.vsc[0] >> (8 * pi)) * vm);
        } else {
          vs = bits2half((uint16_t)(cv.vsc[pi >> 1] >> (16 * (pi & 1))));
        }
        s_vs[w][(pi * NCG + gi) * 16 + ln] = half2bits(vs);
      }
      load_vscale(cv, p0 + 16);
    }

    __builtin_amdgcn_sched_barrier(0);  // phases stay apart: bounds the live registers
    // ---- S = K_hat q on 4x4x4 blocks
    float4_t sa0 = {0.f, 0.f, 0.f, 0.f}, sa1 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KV) {
#pragma unroll
      for (int s = 0; s < NS4; ++s) {
        const half2_t c0 = code_pair<BITS, D, BITS>(kx.kw, 2 * s);
        const half2_t c1 = code_pair<BITS, D, BITS>(kx.kw, 2 * s + 1);
        const half4_t ak = {c0[0], c0[1], c1[0], c1[1]};
        const half4_t bh = *reinterpret_cast<const half4_t*>(sq4 + (s * 4 + sc) * 4);
        const half4_t bl = *reinterpret_cast<const half4_t*>(sq4lo + (s * 4 + sc) * 4);
        sa0 = mfma4x4(ak, bh, sa0);
        sa1 = mfma4x4(ak, bl, sa1);
      }
    } else {
      _Float16 ksg[NCG];
      {
        const float km = SM == 1 ? h2f((uint16_t)__shfl(cmeta, (lane & 48) + 10, 64)) : 0.f;
#pragma unroll
        for (int g = 0; g < NCG; ++g) {
          if constexpr (SM == 1) ksg[g] = (_Float16)((float)(int8_t)(kx.ksc[0] >> (8 * g)) * km);
          else ksg[g] = bits2half((uint16_t)(kx.ksc[g >> 1] >> (16 * (g & 1))));
        }
      }
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
    }

    load_k(p0 + 16);  // the next window's K rows and metadata, while this window runs
    meta_nx = load_meta(p0 + 16);
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax over the window (lane: tokens 4*sbk+i of page lj, query sc)
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = KV ? (sa0[i] + sa1[i]) * s_back : sa0[i] + sa1[i];
      x[i] = (4 * sbk + i < my_nv) ? sv * sm_log2 : -INFINITY;
    }
    if (a.xbuf && corr && sc < GQ && my_nv > 0) {  // logits for the proxy's margins / the entropy
      typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(
          u4_t{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])}, rs_ws,
          vo_x, so_x + (uint32_t)p0 * 64u, 0);
    }
    const float mx = fkey_inv(pair32_max_i(pair16_max_i(row4_max_i(fkey(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])))))));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;  // a window with no valid token so far
    const float f_old = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
    float lsum = (e[0] + e[1]) + (e[2] + e[3]);
    if constexpr (KV) {  // L over the fp16 weights the V product and the apply pass use
      lsum = ((float)(_Float16)e[0] + (float)(_Float16)e[1]) + ((float)(_Float16)e[2] + (float)(_Float16)e[3]);
    }
    l_run = l_run * f_old + pair32_sum(pair16_sum(row4_sum(lsum)));
    if (__builtin_expect(__any(f_old != 1.f), 0)) {
#pragma unroll
      for (int h = 0; h < D / 64; ++h) oacc[h] *= f_old;  // the lane's own query
#pragma unroll
      for (int g = 0; g < NCG; ++g) wsum[g] *= f_old;
    }
    const uint32_t e01 = pack_h2(e[0], e[1]), e23 = pack_h2(e[2], e[3]);
    lds_sync_wave();  // the V scales of the window
    {
      half2_t eh01, eh23;
      __builtin_memcpy(&eh01, &e01, 4);
      __builtin_memcpy(&eh23, &e23, 4);
#pragma unroll
      for (int g = 0; g < NCG; ++g) {
        const uint2 sv = *reinterpret_cast<const uint2*>(&s_vs[w][(lj * NCG + g) * 16 + 4 * sbk]);
        half2_t s01, s23;
        __builtin_memcpy(&s01, &sv.x, 4);
        __builtin_memcpy(&s23, &sv.y, 4);
        if constexpr (KV) {
          float pf[4] = {(float)eh01[0] * (float)s01[0], (float)eh01[1] * (float)s01[1],
                         (float)eh23[0] * (float)s23[0], (float)eh23[1] * (float)s23[1]};  // exact
          const half2_t h01 = {(_Float16)pf[0], (_Float16)pf[1]}, h23 = {(_Float16)pf[2], (_Float16)pf[3]};
          const half2_t l01 = {(_Float16)(pf[0] - (float)h01[0]), (_Float16)(pf[1] - (float)h01[1])};
          const half2_t l23 = {(_Float16)(pf[2] - (float)h23[0]), (_Float16)(pf[3] - (float)h23[1])};
          wsum[g] += (pf[0] + pf[1]) + (pf[2] + pf[3]);
          pwg_store<NCG>(s_pw[w], g, h2bits(h01), h2bits(h23), lane);
          pwg_store<NCG>(s_pwl[w], g, h2bits(l01), h2bits(l23), lane);
        } else {
          const half2_t p01 = eh01 * s01, p23 = eh23 * s23;
          wsum[g] = __builtin_amdgcn_fdot2(p01, one2, wsum[g], false);
          wsum[g] = __builtin_amdgcn_fdot2(p23, one2, wsum[g], false);
          pwg_store<NCG>(s_pw[w], g, h2bits(p01), h2bits(p23), lane);
        }
      }
    }

    __builtin_amdgcn_sched_barrier(0);
    if (corr) {
    // ---- page records: m_ref, K-slot moments, V-block masses (this lane:
    // page lj, query sc; the lanes with sbk == 0 write)
    const int my_page = p0 + lj;
    const bool rec_lane = sc < GQ && my_meta != 0 && my_nv > 0;
    const uint32_t so_rp = so_rec + (uint32_t)(p0 * a.F) * 4u;  // the window's part of the offsets is uniform
    if (rec_lane && sbk == 0) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_new), rs_ws, vo_rec, so_rp, 0);
    // t*: the first token of largest e of page lj for query sc (istar: its
    // index among the lane's 4 tokens, out of range in the other lanes)
    int istar = -1;
    if (mom) {
      // e >= 0: the integer order of the bits is the float order
      const float emax = __int_as_float(row4_max_i(max(max(__float_as_int(e[0]), __float_as_int(e[1])),
                                                       max(__float_as_int(e[2]), __float_as_int(e[3])))));
      int fi = 4;
#pragma unroll
      for (int i = 3; i >= 0; --i)
        if (e[i] == emax) fi = i;
      istar = row4_min_i(fi < 4 ? 4 * sbk + fi : 16) - 4 * sbk;
      if (rec_lane && sbk == 0)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(emax), rs_ws, vo_rec,
                                              so_rp + (uint32_t)(1 + 4 * a.k_cap) * 4u, 0);
    }
    if (rec_lane)
      __builtin_amdgcn_raw_buffer_store_b64(u2_t{e01, e23}, rs_ws,
                                            vo_e, so_e + (uint32_t)p0 * 32u, 0);
    const uint32_t vmask = (uint32_t)(vbal >> (16 * lj + 6)) & 0xfu;
    uint32_t kmask = kmask0;  // stored slots past k_cap are not scored (the select kernel flags them)
    for (int r = 0; mom && r < a.k_cap; ++r) {
      const bool has = kmask != 0u;
      if (!__any(has)) break;
      const int cgr = has ? (int)__builtin_ctz(kmask) : 0;  // the r-th stored channel group
      kmask &= kmask - 1u;
      uint32_t rw[4], kscr;
      if (r == 0) {
        rw[0] = rw0[0]; rw[1] = rw0[1]; rw[2] = rw0[2]; rw[3] = rw0[3];
        kscr = ksc0;
        // the scale is read here, not at the top of the window where its load
        // was just issued (a conversion there would wait for it)
        asm volatile("" : "+v"(kscr));
      } else {
        const int slotr = __shfl(cmeta, (lane & 48) + 2 + cgr, 64);
        const uint32_t soff = has ? (uint32_t)slotr : 0u;  // lanes without a slot read slot 0 and drop it
        const uint4 v = ld_off<uint4>(kres_row, soff * G::KSB + ln * 16);
        rw[0] = v.x; rw[1] = v.y; rw[2] = v.z; rw[3] = v.w;
        kscr = ld_off<uint16_t>(kres_sc, soff * 2u);
      }
      float4_t racc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const half2_t c0 = code_pair<4, 32, 4>(rw, 2 * s);
        const half2_t c1 = code_pair<4, 32, 4>(rw, 2 * s + 1);
        const half4_t ar = {c0[0], c0[1], c1[0], c1[1]};
        const half4_t bq = *reinterpret_cast<const half4_t*>(sqr4 + ((cgr * 8 + s) * 4 + sc) * 4);
        racc = mfma4x4(ar, bq, racc);
      }
      // moments of u = racc * e over the tokens other than t* (dS = racc *
      // f scales them by f^2), and D* = racc_t*^2
      // t*'s terms enter as exact zeros (the sums are non-negative, so
      // adding +0 changes no bit), which keeps the loop free of branches
      float M2 = 0.f, M3 = 0.f, M4 = 0.f, Ds = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool st = i == istar;
        const float r2 = racc[i] * racc[i];
        const float u = st ? 0.f : racc[i] * e[i];
        const float ue = st ? 0.f : u * e[i];
        M2 = fmaf(u, u, M2);
        M3 = fmaf(ue, u, M3);
        M4 = fmaf(ue, ue, M4);
        Ds = st ? r2 : Ds;
      }
      M2 = row4_sum(M2); M3 = row4_sum(M3); M4 = row4_sum(M4); Ds = row4_sum(Ds);
      if (has && rec_lane && sbk == 0) {
        const float f = h2f((uint16_t)kscr) * a.inv_sqrt_d;
        const float f2 = f * f;
        const uint32_t o = so_rp + (uint32_t)(1 + 4 * r) * 4u;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M2 * f2), rs_ws, vo_rec, o, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M3 * f2), rs_ws, vo_rec, o + 4u, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M4 * f2), rs_ws, vo_rec, o + 8u, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Ds * f2), rs_ws, vo_rec, o + 12u, 0);
      }
    }
    // V block sbk of page lj: its stored-slot rank and mass
    if (rec_lane && ((vmask >> sbk) & 1u)) {
      const int vrank = (int)__builtin_popcount(__builtin_amdgcn_ubfe(vmask, 0u, (uint32_t)sbk));  // blocks before sbk
      if (vrank < a.v_cap)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint((e[0] + e[1]) + (e[2] + e[3])), rs_ws,
                                              vo_rec + (uint32_t)vrank * 4u, so_rp + (uint32_t)(2 + 4 * a.k_cap) * 4u, 0);
    }
    }  // records
    __builtin_amdgcn_sched_barrier(0);
    // ---- O += P V_hat, page by page
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      const bool live = nvp[pi] > 0;
      if (live) {
        uint32_t vp[CH / 2];
#pragma unroll
        for (int i = 0; i < CH / 2; ++i) {
          if constexpr (KV) {  // exact signed codes: no offset to take back
            const half2_t c = code_pair<BITS, CH, BITS>(cv.vw[pi], i);
            vp[i] = h2bits(c);
          } else {
            vp[i] = code_pair_sub<BITS, CH, BITS>(cv.vw[pi], i);
          }
        }
        vtile_write_raw<D, BITS>(vt, vp, ln, lj);
      }
      load_vpage(cv, p0 + 16, pi);  // the next window's page pi into the registers just consumed
      if (!live) continue;
      lds_sync_wave();
#pragma unroll
      for (int h = 0; h < D / 64; ++h) {
        uint2 pg[4];  // P'[query sc][tokens g, g+4, g+8, g+12] of page pi, the lane's group
        pwg_load<NCG>(s_pw[w], pi, 2 * h + (lane >> 5), sc, pg);
#pragma unroll
        for (int g = 0; g < 4; ++g) pv4_step<D, BITS>(vt, g, h, pg[g].x, pg[g].y, oacc[h], lane);
        if constexpr (KV) {
          pwg_load<NCG>(s_pwl[w], pi, 2 * h + (lane >> 5), sc, pg);
#pragma unroll
          for (int g = 0; g < 4; ++g) pv4_step<D, BITS>(vt, g, h, pg[g].x, pg[g].y, oacc[h], lane);
        }
      }
      lds_sync_wave();
    }
  }

  // weight sums per (query, group) over the wave: lanes l with l % 4 = q
  float bias[D / 64];
  {
#pragma unroll
    for (int g = 0; g < NCG; ++g) wsum[g] = col_sum(row4_sum(wsum[g]));
#pragma unroll
    for (int h = 0; h < D / 64; ++h) {
      float lo = wsum[2 * h], hi = wsum[2 * h + 1];
      asm volatile("" : "+v"(lo), "+v"(hi));  // a select of values, not of array slots
      bias[h] = (lane >> 5) ? hi : lo;
    }
  }
  if constexpr (KV)
    merge4_waves<D, BITS>(reinterpret_cast<float*>(smem), s_m, s_l, m_run, l_run, oacc, w, lane, GQ,
                          a.po + ((long)bk * a.nsplit + split) * 16 * D, a.pml + ((long)bk * a.nsplit + split) * 16 * 2);
  else
    merge4_waves_raw<D, BITS>(reinterpret_cast<float*>(smem), s_m, s_l, m_run, l_run, oacc, bias, w, lane, GQ,
                             a.po + ((long)bk * a.nsplit + split) * 16 * D,
                             a.pml + ((long)bk * a.nsplit + split) * 16 * 2);
}

int launch_decode_stream4(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit_run, A.n_kv_heads, a.B);
  if (a.split_base != 0 || a.range != (A.kivi_packed ? 1 : 0)) {
    set_error("decode_stream4: runs the whole row of a uniform base or the packed KIVI prefix from split 0");
    return CAREKV_EINVAL;
  }
  if (A.kivi_packed) {
    if (A.base_bits != 2 || A.scale_mode != 0) {
      set_error("decode_stream4: a packed KIVI arena has base_bits 2 and scale_mode 0");
      return CAREKV_EINVAL;
    }
    if (A.head_dim == 64) hipLaunchKernelGGL((decode_stream4_kernel<64, 2, 0, true>), grid, dim3(256), 0, s, A, a);
    else if (A.head_dim == 128) hipLaunchKernelGGL((decode_stream4_kernel<128, 2, 0, true>), grid, dim3(256), 0, s, A, a);
    else {
      set_error("decode_stream4: head_dim %d (kernels: 64, 128)", A.head_dim);
      return CAREKV_EINVAL;
    }
    CAREKV_CHECK_LAUNCH("decode_stream4 (packed KIVI)");
    return CAREKV_OK;
  }
  return dispatch_dbs(A.head_dim, A.base_bits, A.scale_mode, [&](auto d, auto bb, auto sm) {
    hipLaunchKernelGGL((decode_stream4_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value>), grid,
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_stream4");
    return CAREKV_OK;
  });
}

}  // namespace carekv
