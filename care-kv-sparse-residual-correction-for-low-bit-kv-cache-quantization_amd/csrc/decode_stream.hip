// Streaming pass of the CARE-KV decode: one work-group per (split of pages,
// kv head, sequence), 4 waves, one 16-token page per wave iteration.
//
// Per page (lane l: m = l % 16, j = l / 16):
//   * K and V codes of token m, dims [j*D/4, (j+1)*D/4) are dequantised
//     exactly, half(code * scale) (quantizer.py:67-82; int8 scale codes read
//     back as half(code * master), cache.py:713-718), two codes at a time:
//     a packed field pair is masked into the mantissas of two fp16 values
//     1024 + u*2^p (u = offset-binary code), one packed FMA recovers the two
//     signed codes exactly, one packed multiply applies the scale with a
//     single round-to-nearest-even.  The pairing fixes the order of the
//     reduction dimension; q is loaded in the same order.
//   * S = K_hat q for all query heads of the GQA group on MFMA 16x16x16 f16
//     (rows: tokens, columns: query heads), online softmax in fp32.
//   * O += P V_hat on MFMA, V_hat transposed through LDS.
//   * For every stored K slot: dS = q_cg R_K / sqrt(D) on MFMA and the
//     moments sum dS^2 e^k (k = 2, 3, 4) of e = exp(s - m_ref); for every
//     stored V slot the block mass sum e.  These give the query-aware K score
//     (attention.py:167-184) and V score (attention.py:788-790) once the
//     global softmax statistics are known (finalize kernel).
// The next page's codes, scales and slot tables are loaded while the
// current page is processed.
#include "decode_common.h"
#include "host_util.h"

namespace carekv {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- unpack schedule
// Codes are pair-wise (k, k + PD) inside blocks of BLK codes.
template <int BITS> struct PairGeom;
template <> struct PairGeom<2> { static constexpr int BLK = 16, PD = 8; };
template <> struct PairGeom<3> { static constexpr int BLK = 8, PD = 4; };
template <> struct PairGeom<4> { static constexpr int BLK = 8, PD = 4; };

template <int BITS, int NC>
struct Unpack {
  static constexpr int NP = NC / 2;
  static constexpr int NW = (NC * BITS + 31) / 32;
  struct Tab {
    int a[NP], b[NP], W[NP], ao[NP], bo[NP];
    uint32_t xr[NW];
    int slot_code[NC];  // slot e (2i + half) -> code index within the chunk
  };
  static constexpr Tab make() {
    Tab t{};
    constexpr int BLK = PairGeom<BITS>::BLK, PD = PairGeom<BITS>::PD, MAXO = 10 - BITS;
    int n = 0;
    for (int blk = 0; blk < NC; blk += BLK)
      for (int k = 0; k < BLK / 2; ++k) {
        const int ia = blk + k, ib = ia + PD;
        const int ba = BITS * ia, bb = BITS * ib;
        int lo = ba - MAXO, hi = ba;
        if (bb - 16 - MAXO > lo) lo = bb - 16 - MAXO;
        if (bb - 16 < hi) hi = bb - 16;
        int W = hi;
        for (int c = hi; c >= lo; --c)
          if (c >= 0 && c % 32 == 0) { W = c; break; }
        t.a[n] = ia; t.b[n] = ib; t.W[n] = W; t.ao[n] = ba - W; t.bo[n] = bb - W - 16;
        t.slot_code[2 * n] = ia; t.slot_code[2 * n + 1] = ib;
        ++n;
      }
    for (int k = 0; k < NC; ++k) {  // two's complement -> offset binary: flip each field's top bit
      const int bit = BITS * k + BITS - 1;
      t.xr[bit / 32] |= 1u << (bit % 32);
    }
    return t;
  }
  static constexpr Tab T = make();
};

// 32-bit window of the code bit string starting at bit W (W may be negative).
template <int BITS, int NC>
__device__ __forceinline__ uint32_t window(const uint32_t* w, int W, int hi_bit) {
  if (W < 0) return w[0] << (-W);
  const int d = W / 32, s = W % 32;
  if (s == 0) return w[d];
  if (hi_bit < 32 * (d + 1)) return w[d] >> s;
  return __builtin_amdgcn_alignbit(w[d + 1], w[d], s);
}

// Exact half(code*s) for NC codes (two's complement, LE bit string in w,
// w is modified) as NC/2 fp16 pairs (codes a_i, b_i of the schedule).
template <int BITS, int NC>
__device__ __forceinline__ void unpack_pairs(uint32_t* w, _Float16 s, half2_t* out) {
  using U = Unpack<BITS, NC>;
#pragma unroll
  for (int i = 0; i < U::NW; ++i) w[i] ^= U::T.xr[i];
  const half2_t ss = {s, s};
  constexpr uint32_t fmask = (1u << BITS) - 1u;
#pragma unroll
  for (int i = 0; i < U::NP; ++i) {
    const int W = U::T.W[i], ao = U::T.ao[i], bo = U::T.bo[i];
    uint32_t x = window<BITS, NC>(w, W, BITS * U::T.b[i] + BITS - 1);
    x = (x & ((fmask << ao) | (fmask << (16 + bo)))) | 0x64006400u;
    half2_t v;
    __builtin_memcpy(&v, &x, 4);
    const half2_t sc = {(_Float16)(1.0f / (float)(1 << ao)), (_Float16)(1.0f / (float)(1 << bo))};
    const half2_t of = {(_Float16)(-(1024.0f / (float)(1 << ao) + (float)(1 << (BITS - 1)))),
                        (_Float16)(-(1024.0f / (float)(1 << bo) + (float)(1 << (BITS - 1))))};
    const half2_t c = __builtin_elementwise_fma(v, sc, of);  // exact signed codes
    out[i] = c * ss;                                          // one RNE rounding each
  }
}

__device__ __forceinline__ uint32_t h2bits(half2_t v) {
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

template <int D, int BITS>
__global__ __launch_bounds__(256) void decode_stream_kernel(carekv_arena A, DecodeArgs a) {
  constexpr int NT = D / 16;           // MFMA k-steps for S; PV output tiles
  constexpr int CH = D / 4;            // codes per lane (one quarter of a row)
  constexpr int CHB = CH * BITS / 8;   // packed bytes per lane
  constexpr int NWC = (CHB + 3) / 4;   // 32-bit words per lane chunk
  constexpr int RB = row_bytes(D, BITS);
  constexpr int NCG = D / 32;
  constexpr int KSB = kPage * 32 / 2;
  using U = Unpack<BITS, CH>;

  constexpr int LDS_BYTES = 4 * 16 * D * 4;  // merge buffer; the V tiles use the first half
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ float s_m[4][16], s_l[4][16];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int Hkv = A.n_kv_heads, GQ = a.GQ;
  const int bk = b * Hkv + kvh;
  const int seq_raw = a.seq_slot[b], np_raw = a.n_pages[b];
  const bool row_ok = seq_raw >= 0 && seq_raw < A.n_seq && np_raw >= 0 && np_raw <= a.Pmax;
  const int seq = row_ok ? seq_raw : 0, np = row_ok ? np_raw : 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ln = lane & 15, lj = lane >> 4;
  const long pg_base = ((long)kvh * A.n_seq + seq) * A.max_pages;
  const int F = a.F;
  const int gi = (lj * CH) / 32;  // quant group of this lane's chunk

  // ---- B operands.  S step s uses codes (a_2s, b_2s, a_2s+1, b_2s+1) of the
  // lane's chunk; lane (n = query, j) holds q_n at those dims.  qR[cg][s]:
  // q_n[cg*32 + 8j + 4s + i] for the dS product with the 4-bit K slot rows.
  half4_t qB[NT], qR[NCG][2];
  {
    const bool qv = ln < GQ;
    const uint16_t* qp = a.q + ((long)b * a.Hq + kvh * GQ + (qv ? ln : 0)) * D;
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const int c0 = lj * CH;
      qB[s][0] = qv ? bits2half(qp[c0 + U::T.a[2 * s]]) : (_Float16)0.f;
      qB[s][1] = qv ? bits2half(qp[c0 + U::T.b[2 * s]]) : (_Float16)0.f;
      qB[s][2] = qv ? bits2half(qp[c0 + U::T.a[2 * s + 1]]) : (_Float16)0.f;
      qB[s][3] = qv ? bits2half(qp[c0 + U::T.b[2 * s + 1]]) : (_Float16)0.f;
    }
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) qR[cg][s][i] = qv ? bits2half(qp[cg * 32 + 8 * lj + 4 * s + i]) : (_Float16)0.f;
  }

  uint32_t* vt = reinterpret_cast<uint32_t*>(smem) + w * kPage * (D / 2);  // this wave's V tile, pairs
  float m_run = -INFINITY, l_run = 0.f;
  float4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int p_begin = split * a.SP, p_end = min(p_begin + a.SP, np);

  // ---- prefetched page state
  uint32_t kw[NWC + 1], vw[NWC + 1];
  int ksc = 0, vsc = 0, nvld = 0, meta = 0;
  float kmast = 0.f, vmast = 0.f;
  int ksl[NCG], vsl[kVtb];
  auto load_page = [&](int p, uint32_t* kwo, uint32_t* vwo, int& kso, int& vso, float& kmo, float& vmo, int& nvo,
                       int& meo, int* kslo, int* vslo) {
    const long pg = pg_base + p;
    kwo[NWC] = 0; vwo[NWC] = 0;
    load_bytes<CHB>(kwo, A.kcodes + (pg * kPage + ln) * RB + lj * CHB);
    load_bytes<CHB>(vwo, A.vcodes + (pg * kPage + ln) * RB + lj * CHB);
    if (A.scale_mode == 1) {
      kso = ((const int8_t*)A.kscale)[(pg * kPage + ln) * NCG + gi];
      vso = ((const int8_t*)A.vscale)[(pg * kPage + ln) * NCG + gi];
      kmo = h2f(A.kmaster[pg]);
      vmo = h2f(A.vmaster[pg]);
    } else {
      kso = ((const uint16_t*)A.kscale)[(pg * kPage + ln) * NCG + gi];
      vso = ((const uint16_t*)A.vscale)[(pg * kPage + ln) * NCG + gi];
    }
    nvo = A.valid[pg];
    meo = A.has_meta[pg];
#pragma unroll
    for (int c = 0; c < NCG; ++c) kslo[c] = A.k_slot[pg * NCG + c];
#pragma unroll
    for (int v = 0; v < kVtb; ++v) vslo[v] = A.v_slot[pg * kVtb + v];
  };
  int p = p_begin + w;
  if (p < p_end) load_page(p, kw, vw, ksc, vsc, kmast, vmast, nvld, meta, ksl, vsl);

  for (; p < p_end; p += 4) {
    // current page state
    uint32_t ckw[NWC + 1], cvw[NWC + 1];
#pragma unroll
    for (int i = 0; i <= NWC; ++i) { ckw[i] = kw[i]; cvw[i] = vw[i]; }
    const int cks = ksc, cvs = vsc, nv = nvld, cmeta = meta;
    const float ckm = kmast, cvm = vmast;
    int cksl[NCG], cvsl[kVtb];
#pragma unroll
    for (int c = 0; c < NCG; ++c) cksl[c] = ksl[c];
#pragma unroll
    for (int v = 0; v < kVtb; ++v) cvsl[v] = vsl[v];
    if (p + 4 < p_end) load_page(p + 4, kw, vw, ksc, vsc, kmast, vmast, nvld, meta, ksl, vsl);
    const long pg = pg_base + p;
    float* rec = a.rec + ((long)bk * a.Pmax + p) * GQ * F;
    if (nv <= 0) {
      if (lj == 0 && ln < GQ) rec[ln * F] = -INFINITY;
      continue;
    }
    // K slot rows of this page (issued early, used after the attention math)
    uint32_t rw[NCG];
    float rsc[NCG];
#pragma unroll
    for (int cg = 0; cg < NCG; ++cg) {
      rw[cg] = 0; rsc[cg] = 0.f;
      if (cmeta && cksl[cg] >= 0) {
        const long so = (long)seq * A.n_slots + cksl[cg];
        rw[cg] = *reinterpret_cast<const uint32_t*>(A.k_res + so * KSB + ln * 16 + lj * 4);
        rsc[cg] = h2f(A.k_res_scale[so]);
      }
    }
    _Float16 ks, vs;
    if (A.scale_mode == 1) {
      ks = (_Float16)((float)cks * ckm);
      vs = (_Float16)((float)cvs * cvm);
    } else {
      ks = bits2half((uint16_t)cks);
      vs = bits2half((uint16_t)cvs);
    }
    // ---- S = K_hat q
    half2_t kp[CH / 2];
    unpack_pairs<BITS, CH>(ckw, ks, kp);
    float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NT; ++s) {
      const half4_t ak = {kp[2 * s][0], kp[2 * s][1], kp[2 * s + 1][0], kp[2 * s + 1][1]};
      sacc = mfma16(ak, qB[s], sacc);
    }
    // V_hat pairs to LDS while the softmax runs
    {
      half2_t vp[CH / 2];
      unpack_pairs<BITS, CH>(cvw, vs, vp);
      uint32_t* dst = vt + ln * (D / 2) + lj * (CH / 2);
#pragma unroll
      for (int i = 0; i < CH / 2; i += 4) {
        *reinterpret_cast<uint4*>(dst + i) = make_uint4(h2bits(vp[i]), h2bits(vp[i + 1]), h2bits(vp[i + 2]),
                                                        h2bits(vp[i + 3]));
      }
    }
    // lane (n = query, j): sacc[i] = S[token 4j+i][query n]
    float sv[4], e[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = (4 * lj + i < nv) ? sacc[i] * a.sm_scale : -INFINITY;
      mx = fmaxf(mx, sv[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    float f_old = 1.f;
    if (m_new > m_run) f_old = (m_run == -INFINITY) ? 0.f : expf(m_run - m_new);
    m_run = m_new;
    float esum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = (4 * lj + i < nv) ? expf(sv[i] - m_run) : 0.f;
      esum += e[i];
    }
    esum += __shfl_xor(esum, 16, 64);
    esum += __shfl_xor(esum, 32, 64);
    l_run = l_run * f_old + esum;
    if (__builtin_amdgcn_read_exec() && __any(f_old != 1.f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float fi = __shfl(f_old, 4 * lj + i, 64);
#pragma unroll
        for (int t = 0; t < NT; ++t) oacc[t][i] *= fi;
      }
    }
    const half4_t ap = {(_Float16)e[0], (_Float16)e[1], (_Float16)e[2], (_Float16)e[3]};
    // ---- O += P V_hat.  Tile t, column n stands for V slot n*NT + t.
    lds_sync_wave();
    uint32_t vr[4][NT / 2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t* src = vt + (4 * lj + i) * (D / 2) + ln * (NT / 2);
      if constexpr (NT / 2 == 4) {
        const uint4 x = *reinterpret_cast<const uint4*>(src);
        vr[i][0] = x.x; vr[i][1] = x.y; vr[i][2] = x.z; vr[i][3] = x.w;
      } else {
        const uint2 x = *reinterpret_cast<const uint2*>(src);
        vr[i][0] = x.x; vr[i][1] = x.y;
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int wi = t >> 1;
      const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;  // high / low halves of two words
      const uint32_t p01 = __builtin_amdgcn_perm(vr[1][wi], vr[0][wi], sel);
      const uint32_t p23 = __builtin_amdgcn_perm(vr[3][wi], vr[2][wi], sel);
      half4_t bv;
      __builtin_memcpy(&bv, &p01, 4);
      __builtin_memcpy(reinterpret_cast<char*>(&bv) + 4, &p23, 4);
      oacc[t] = mfma16(ap, bv, oacc[t]);
    }
    lds_sync_wave();

    // ---- record: m_ref, K-slot moments, V-block masses
    if (lj == 0 && ln < GQ) rec[ln * F] = m_run;
    if (cmeta) {
      int rk = 0;
#pragma unroll
      for (int cg = 0; cg < NCG; ++cg) {
        if (cksl[cg] < 0) continue;
        if (rk >= a.k_cap) { if (lane == 0) *a.err_flag = 1; break; }
        half4_t r0, r1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          r0[i] = (_Float16)(float)get_code<4>(&rw[cg], i);
          r1[i] = (_Float16)(float)get_code<4>(&rw[cg], 4 + i);
        }
        float4_t racc = {0.f, 0.f, 0.f, 0.f};
        racc = mfma16(r0, qR[cg][0], racc);
        racc = mfma16(r1, qR[cg][1], racc);
        float M2 = 0.f, M3 = 0.f, M4 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ds = (racc[i] * rsc[cg]) / a.sqrt_d;
          const float y = ds * e[i];
          const float x = y * y;
          const float xe = x * e[i];
          M2 += x;
          M3 += xe;
          M4 += xe * e[i];
        }
        M2 += __shfl_xor(M2, 16, 64); M2 += __shfl_xor(M2, 32, 64);
        M3 += __shfl_xor(M3, 16, 64); M3 += __shfl_xor(M3, 32, 64);
        M4 += __shfl_xor(M4, 16, 64); M4 += __shfl_xor(M4, 32, 64);
        if (lj == 0 && ln < GQ) {
          float* r = rec + ln * F + 1 + 3 * rk;
          r[0] = M2; r[1] = M3; r[2] = M4;
        }
        ++rk;
      }
      int rv = 0, my_slot = -1, my_rank = 0;
#pragma unroll
      for (int vb = 0; vb < kVtb; ++vb) {
        if (vb == lj) { my_slot = cvsl[vb]; my_rank = rv; }
        rv += cvsl[vb] >= 0;
      }
      if (my_slot >= 0 && ln < GQ) {
        if (my_rank < a.v_cap) rec[ln * F + 1 + 3 * a.k_cap + my_rank] = e[0] + e[1] + e[2] + e[3];
        else *a.err_flag = 1;
      }
    }
  }

  // ---- merge the 4 waves' (m, l, O) and write the split partial; V slot
  // n*NT + t maps back to dim chunk*CH + slot_code[slot % CH].
  float* so = reinterpret_cast<float*>(smem);  // [4][16][D]
  __syncthreads();
  if (lj == 0) { s_m[w][ln] = m_run; s_l[w][ln] = l_run; }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int slot = ln * NT + t;
    const int dim = (slot / CH) * CH + U::T.slot_code[slot % CH];
#pragma unroll
    for (int i = 0; i < 4; ++i) so[(w * 16 + 4 * lj + i) * D + dim] = oacc[t][i];
  }
  __syncthreads();
  const long pbase = ((long)bk * a.nsplit + split) * 16;
  for (int idx = threadIdx.x; idx < GQ * D; idx += 256) {
    const int qq = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][qq]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float f = s_m[ww][qq] == -INFINITY ? 0.f : expf(s_m[ww][qq] - M);
        L += s_l[ww][qq] * f;
        O += so[(ww * 16 + qq) * D + d] * f;
      }
    }
    a.po[(pbase + qq) * D + d] = O;
    if (d == 0) { a.pml[(pbase + qq) * 2] = M; a.pml[(pbase + qq) * 2 + 1] = L; }
  }
}

int launch_decode_stream(const carekv_arena& A, const DecodeArgs& a, hipStream_t s) {
  dim3 grid(a.nsplit, A.n_kv_heads, a.B);
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto bb) {
    hipLaunchKernelGGL((decode_stream_kernel<decltype(d)::value, decltype(bb)::value>), grid, dim3(256), 0, s, A, a);
    CAREKV_CHECK_LAUNCH("decode_stream");
    return CAREKV_OK;
  });
}

}  // namespace carekv
