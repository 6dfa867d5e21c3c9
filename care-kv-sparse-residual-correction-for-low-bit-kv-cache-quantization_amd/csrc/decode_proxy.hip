// Page terms of the sketch-proxy K score (CAREKV_KSCORE_LIVE=0): between the
// streaming and select kernels, one work-group per (split of pages, kv head,
// sequence).  For every query head of the GQA group and every page with a
// stored K slot, over the page's valid tokens t (attention.py:718-725, the
// same terms as ResidualRouter.route, residual_router.py:160-170):
//   mass     = sum_t a_t
//   boundary = sum_t a_t * (1 / max(s_top - s_t, 1e-6))
//   vdiff    = sum_t a_t * ||V_hat_t - O_base||
// with a = softmax(s) over the whole context, s_top = max_t s_t and O_base
// the fp32 base output.  The logits are the streaming kernel's own (x =
// s log2(e) in xbuf), so s_top is the maximum of exactly the values the
// margins subtract; a_t = 2^(x_t - M) / L from the split statistics; V_hat
// is dequantised exactly as in the streaming pass.
//
// Lane l = 16 j + m: token m, dims [j D/4, (j+1) D/4) of the page for the
// distance sums; afterwards the 16 lanes of row j finish query 4 k + j.
//
// PF (prefill rows, the per-(head, row) router of correction_impl=cached,
// layer.py:573-640): a is the reference's fp16 attention weight of the row
// (the streaming pass's stored weights, against the row's log-sum-exp),
// s_top the row's largest logit (the streaming pass's per-wave maxima),
// O_base the fp16 base output half(sum_t a_t V_hat_t) (layer.py:964-965),
// V_hat the prompt's dense fp16 rows; logits past the row are -inf and
// their weights 0.
#include "decode_page.h"
#include "host_util.h"

namespace carekv {

__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int D, int BITS, int SM, bool PF = false>
__global__ __launch_bounds__(256) void decode_proxy_kernel(carekv_arena A, DecodeArgs a) {
  using G = PageGeom<D, BITS>;
  using PB = typename G::PB;
  constexpr int NCG = G::NCG, CH = G::CH, CHB = G::CHB, RB = G::RB, NWC = G::NWC;
  constexpr float kEps = 1e-6f;               // residual_router.py:34
  constexpr float kLn2 = 0.693147180559945f;  // margins back from base-2 logits
  __shared__ float s_o[16 * D];               // O_base [query][dim]
  __shared__ float s_M[16], s_L[16], s_Mp[16];

  // prefill rows: the latest (longest) rows first
  const int split = blockIdx.x, kvh = blockIdx.y, b = a.pf ? (int)(gridDim.z - 1 - blockIdx.z) : (int)blockIdx.z;
  const int GQ = a.GQ;
  const int bk = b * A.n_kv_heads + kvh;
  const EntryRow er = entry_row(A, a, b);
  const int seq = er.seq, np = er.np;
  int p_lo, p_hi;
  launch_pages(A, a, seq, np, p_lo, p_hi);
  const int p_begin = p_lo + split * a.SP, p_end = min(p_begin + a.SP, p_hi);
  if (p_begin >= p_end) return;  // uniform over the work-group
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15, lj = lane >> 4;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;

  // ---- softmax statistics and O_base of the group's queries (split order)
  if ((int)threadIdx.x < GQ) {
    const int qq = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, a.pml[(((long)bk * a.nsplit + s) * 16 + qq) * 2]);
    float L = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < a.nsplit; ++s) {
        const long base = ((long)bk * a.nsplit + s) * 16 + qq;
        const float ms = a.pml[base * 2];
        if (ms != -INFINITY) L += a.pml[base * 2 + 1] * __builtin_amdgcn_exp2f(ms - M);
      }
    float xm = -INFINITY;
    if constexpr (PF)
      for (int i = 0; i < a.nsplit * 4; ++i) xm = fmaxf(xm, a.xmax[((long)bk * a.nsplit * 4 + i) * 16 + qq]);
    s_M[qq] = PF ? xm : M;  // the margins' s_top
    s_L[qq] = L;
    s_Mp[qq] = M;           // the split partials' reference maximum
  }
  __syncthreads();
  for (int i = threadIdx.x; i < GQ * D; i += 256) {
    const int qq = i / D, d = i % D;
    const float M = s_Mp[qq], L = s_L[qq];
    float O = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < a.nsplit; ++s) {
        const long base = ((long)bk * a.nsplit + s) * 16 + qq;
        const float ms = a.pml[base * 2];
        if (ms != -INFINITY) O += a.po[base * D + d] * __builtin_amdgcn_exp2f(ms - M);
      }
    // prefill rows: the fp16 base output, the weights already normalised
    s_o[i] = PF ? (float)(_Float16)O : (L > 0.f ? O / L : 0.f);
  }
  __syncthreads();

  RowRes rr;
  if constexpr (PF) {
    static_assert(BITS == 16, "prefill rows are fp16");
    rr.vc = make_rsrc(a.pf_v + (long)kvh * a.pf_T * D, (uint32_t)a.pf_T * D * 2);  // rows past the prompt read 0
    rr.kc = rr.ks = rr.vs = make_rsrc(nullptr, 0u);
  } else {
    rr = row_resources<D, BITS, SM>(A, pg_base);
  }
  const float* ob = s_o + lj * CH;
  for (int p = p_begin + w; p < p_end; p += 4) {
    const long pg = pg_base + p;
    const int nv = A.valid[pg];
    if (nv <= 0 || !A.has_meta[pg]) continue;
    bool anyk = false;
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      const int s = A.k_slot[pg * NCG + cg];
      anyk |= s >= 0 && s < A.n_slots;
    }
    if (!anyk) continue;  // no K candidate on the page
    // V_hat of token ln, chunk lj
    uint32_t vw[NWC];
    const uint32_t row = (uint32_t)(p * kPage + ln);
    buf_load<CHB>(vw, rr.vc, row * RB + lj * CHB);
    const int gi = (lj * CH) / 32;
    int vcode;
    if constexpr (SM == 1) vcode = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rr.vs, row * NCG + gi, 0, 0);
    else vcode = __builtin_amdgcn_raw_buffer_load_b16(rr.vs, (row * NCG + gi) * 2, 0, 0);
    const float vm = SM == 1 ? h2f(A.vmaster[pg]) : 0.f;
    half2_t vp[CH / 2];
    dequant_pairs<BITS, CH, BITS>(vw, lane_scale<SM>(vcode, vm), vp);

    for (int q0 = 0; q0 < GQ; q0 += 4) {
      // ||V_hat_t - O_q||^2 for queries q0 .. q0+3; row j keeps query q0 + j
      float d2 = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (q0 + u >= GQ) break;
        const float* o = ob + (q0 + u) * D;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CH / 2; ++i) {
          const float d0 = (float)vp[i][0] - o[PB::T.a[i]];
          const float d1 = (float)vp[i][1] - o[PB::T.b[i]];
          acc = fmaf(d0, d0, acc);
          acc = fmaf(d1, d1, acc);
        }
        const float tot = col_sum(acc);
        if (lj == u) d2 = tot;
      }
      const int qq = q0 + lj;
      float at = 0.f, bt = 0.f, vt = 0.f;
      if (qq < GQ && ln < nv) {
        const float M = s_M[qq], L = s_L[qq];
        const float x = a.xbuf[(((long)bk * GQ + qq) * a.Pmax + p) * 16 + ln];
        if (x != -INFINITY && M != -INFINITY && L > 0.f) {
          if constexpr (PF) at = h2f(a.ebuf[(((long)bk * GQ + qq) * a.Pmax + p) * 16 + ln]);
          else at = __builtin_amdgcn_exp2f(x - M) / L;
          bt = at * (1.f / fmaxf((M - x) * kLn2, kEps));
          vt = at * sqrtf(d2);
        }
      }
      at = row16_sum(at);
      bt = row16_sum(bt);
      vt = row16_sum(vt);
      if (qq < GQ && ln == 0)
        *reinterpret_cast<float4*>(a.prox + (((long)bk * GQ + qq) * a.Pmax + p) * 4) = make_float4(at, bt, vt, 0.f);
    }
  }
}

int launch_decode_proxy(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  const dim3 grid(a.nsplit_run, A.n_kv_heads, a.B);
  if (a.pf) {
    if (A.head_dim == 64) hipLaunchKernelGGL((decode_proxy_kernel<64, 16, 0, true>), grid, dim3(256), 0, s, A, a);
    else hipLaunchKernelGGL((decode_proxy_kernel<128, 16, 0, true>), grid, dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_proxy (prefill rows)");
    return CAREKV_OK;
  }
  return dispatch_dbs16(A.head_dim, A.base_bits, A.scale_mode, [&](auto d, auto bb, auto sm) {
    hipLaunchKernelGGL((decode_proxy_kernel<decltype(d)::value, decltype(bb)::value, decltype(sm)::value>), grid,
                       dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_proxy");
    return CAREKV_OK;
  });
}

}  // namespace carekv
