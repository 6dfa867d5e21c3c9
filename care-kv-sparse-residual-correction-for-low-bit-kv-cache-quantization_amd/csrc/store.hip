// Page writes (quantize + pack + int8 page scales), store-time residual
// candidates / selection / slot packing, and single-token decode appends.
//
// Reference semantics (paths relative to the reference root):
//   quantize (fp16 arithmetic)        quantizer.py:31-64
//   INT2/3/4 packing                  quantizer.py:257-372
//   int8 scale codes + fp16 master    cache.py:592-654, 689-695
//   process_page                      residual_store.py:239-464
//   4-bit residual slot packing       residual_store.py:121-136
//   decode append + store on fill     layer.py:1028-1146
#include "common.h"

namespace carekv {

struct StoreWs {  // per job: [0]=K count, [1]=V count, [2]=K base, [3]=V base
  int32_t* v;
};

// One wave quantizes one row group: 32 fp16 values -> codes, fp16 scale.
// fp16 chain of quantizer.py:51-59: max|x| (exact), scale=half(max/qmax),
// code=clamp(rint(half(x/scale))), NaN (0/0 on an all-zero group) -> 0.
template <int BITS>
__device__ __forceinline__ _Float16 quant_group(const float* x, int* code) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(x[i]));
  const _Float16 scale = (_Float16)(m / (float)qmax);
  const float sf = (float)scale;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float qh = (float)(_Float16)(x[i] / sf);
    float r = rintf(qh);
    r = fminf(fmaxf(r, (float)(-qmax - 1)), (float)qmax);
    code[i] = (qh != qh) ? 0 : (int)r;
  }
  return scale;
}

template <int BITS>
__device__ __forceinline__ void pack_group(const int* code, uint32_t* w) {
#pragma unroll
  for (int i = 0; i < BITS; ++i) w[i] = 0;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint32_t u = (uint32_t)code[k] & ((1u << BITS) - 1u);
    const int bit = BITS * k;
    w[bit >> 5] |= u << (bit & 31);
    if ((bit & 31) + BITS > 32) w[(bit >> 5) + 1] |= u >> (32 - (bit & 31));
  }
}

// int8 scale code of `s` against master `m` (cache.py:601-602, 692-693).
__device__ __forceinline__ int8_t scale_code(float s, float m) {
  const float q = s / m;
  if (q != q) return 0;
  return (int8_t)fminf(fmaxf(rintf(q), -128.f), 127.f);
}

// ---------------------------------------------------------------- page store
// One wave stores one page job in a single pass over the page's K and V
// rows (residual_store.py:239-464 after the page write of cache.py:592-654):
// codes, scales and masters, the residuals, the candidate errors and K
// sketches, the store decision, and the 4-bit payloads of the selected
// candidates, which go to a per-job staging area of the workspace.  A scan
// then gives each job its slot ids in call order and a scatter moves the
// staged payloads to their slots.
//
// Lane layout: lane l holds, for chunk i = 0..3, token t = 4 i + l / 16 and
// the EPL = D / 16 channels EPL * (l % 16) .. + EPL - 1 of that token.  A
// chunk is thus one V candidate block (4 tokens), and a quant group (32
// channels of one row) is LPG = 32 / EPL consecutive lanes; a K candidate
// (one 32-channel group over 16 tokens) is the LPG-lane group of every row
// in every chunk.

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int kNvb = kPage / kVtb;  // V candidate blocks per page

enum StorePath : int {
  kPathFresh = 0,    // quantize K / V and write the packed page
  kPathKeep = 1,     // streaming fill store: the page keeps its codes and scales
  kPathCodesIn = 2,  // process_page on the caller's codes and fp16 scales
  kPathKivi = 3,     // packed KIVI prefix page: given 2-bit codes, V scales, K_hat / V_hat
  kPathHat = 4,      // fp16 side-buffer base: given K_hat / V_hat rows
};

template <int D>
struct PageLay {
  static constexpr int EPL = D / 16;              // fp16 values per lane and chunk
  static constexpr int NP = EPL / 2;              // fp16 pairs per lane and chunk
  static constexpr int LPG = kGroup / EPL;        // lanes per quant group
  static constexpr int NG = D / kGroup;           // quant groups (= K candidates) per row
  static constexpr int P = kPage * NG;            // (token, group) pairs per page
  static constexpr int KSB = kPage * kGroup / 2;  // 4-bit K slot bytes
  static constexpr int VSB = kVtb * D / 2;        // 4-bit V slot bytes
};

// LDS of one wave of the store pass.
template <int D>
struct StoreLds {
  uint16_t rk[kPage * D];          // K residual rows (fp16 bits), token-major
  float mean[D];                   // K residual column means
  uint16_t sf[kPage * D / kGroup]; // group scales by (token, group)
  uint16_t svr[kPage * D / kGroup];// V group scales as the decode reads them back
};

// Staged decisions and payloads of one call, in the workspace after the job
// records: per job a header word (bits 0-2 K count, 3-5 V count, 6-8 and
// 9-11 the counts of reused K / V ids, 12-19 and 20-27 the candidate index
// of each K / V selection in slot order, 2 bits each), up to mk K and mv V
// payloads and their fp16 scales (K first).
struct StoreStage {
  uint32_t* head;
  int8_t* kpay;
  int8_t* vpay;
  uint16_t* scale;
  int mk, mv;
};

// Most selections of one kind a page can make under the call's budgets.
__host__ __device__ inline void store_caps(const carekv_store_params& sp, int ng, int* mk, int* mv) {
  if (sp.store_none) {
    *mk = *mv = 0;
    return;
  }
  const int kb = sp.joint ? sp.joint_budget : sp.k_budget;
  const int vb = sp.joint ? sp.joint_budget : sp.v_budget;
  *mk = kb < 0 ? 0 : (kb > ng ? ng : kb);
  *mv = vb < 0 ? 0 : (vb > kNvb ? kNvb : vb);
}

// ---- cross-lane helpers (all 64 lanes active)
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i within 16
constexpr int kDppShl1 = 0x101;        // lane i <- lane i + 1 of its row
constexpr int kDppShl2 = 0x102;        // lane i <- lane i + 2 of its row

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __uint_as_float(dpp_u<CTRL>(__float_as_uint(v)));
}
// Sum / max over aligned N-lane groups of a 16-lane row (N = 1, 2, 4, 8, 16);
// every lane of a group ends with the same bits (the ops commute).
template <int N>
__device__ __forceinline__ float grp_sum(float v) {
  if constexpr (N >= 2) v += dpp_f<kDppXor1>(v);
  if constexpr (N >= 4) v += dpp_f<kDppXor2>(v);
  if constexpr (N >= 8) v += dpp_f<kDppHalfMirror>(v);
  if constexpr (N >= 16) v += dpp_f<kDppMirror>(v);
  return v;
}
template <int N>
__device__ __forceinline__ uint32_t grp_max_u(uint32_t v) {
  if constexpr (N >= 2) v = max(v, dpp_u<kDppXor1>(v));
  if constexpr (N >= 4) v = max(v, dpp_u<kDppXor2>(v));
  if constexpr (N >= 8) v = max(v, dpp_u<kDppHalfMirror>(v));
  if constexpr (N >= 16) v = max(v, dpp_u<kDppMirror>(v));
  return v;
}
// Sum / max over the four rows (lanes c, c+16, c+32, c+48) with the gfx950
// lane swaps: the two halves of each swap hold a pair in some order.
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ uint32_t rows_max_u(uint32_t v) {
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)a[0], (uint32_t)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)b[0], (uint32_t)b[1]);
}

// half(x / s) for the fp16 group scale s > 0 (rc = rcp(s)), the quotient
// of quantizer.py:58.  q1 is one Newton step from x * rc, within 0.5 ulp
// (fp32) plus a 2^-45 relative term of x / s.  x and s are fp16 values, so
// x / s lies no closer than 2^-23 relative (one fp32 ulp) to a midpoint of
// two fp16 values: with odd parts X, S of x, s and an fp16 midpoint m with
// 12-bit odd part M, x = m s would need X = M S >= 2^11, and otherwise
// |x - m s| is at least one unit of m s's last place.  q1 is therefore on
// the same side of every fp16 rounding boundary as x / s, and half(q1) =
// half(x / s), the rounding of the reference's float32 quotient (float32
// carries more than 2 * 11 + 2 bits, so its quotient rounds to fp16 as the
// exact one does).
__device__ __forceinline__ _Float16 quant_q(float x, float s, float rc) {
  // x * rc as an fma with a +0 addend (which takes x as fp16; it differs
  // from the product only in the sign of a zero, which the code drops)
  const float q0 = __builtin_fmaf(x, rc, 0.0f);
  const float e = __builtin_fmaf(-q0, s, x);
  return (_Float16)__builtin_fmaf(e, rc, q0);
}
// The group scale half(m / qmax) (quantizer.py:55) for the fp16 max m: the
// same Newton quotient (m and qmax are fp16 values).
template <int BITS>
__device__ __forceinline__ _Float16 group_scale(float m) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  if constexpr (qmax == 1) {
    return (_Float16)m;
  } else {
    constexpr float rq = 1.0f / (float)qmax;
    return quant_q(m, (float)qmax, rq);
  }
}
// Codes enter the page biased by 1536: for an fp16 q with |q| < 512, the
// fp16 sum q + 1536 lies in [1024, 2048), where fp16 steps by 1, so it is
// 1536 + rint(q) (round half to even: 1536 is even); its bits are
// 0x6600 + code, whose low BITS bits are the code's two's complement.
// With a normal scale s = half(m / qmax) and |x| <= m, |x / s| <= qmax
// (1 + 2^-11) rounds to at most qmax: the clamp binds only for subnormal
// scales (CLAMP).
constexpr float kCodeBias = 1536.f;
template <int BITS, bool CLAMP>
__device__ __forceinline__ h2_t biased_codes(h2_t q) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  const h2_t y = q + h2_t{(_Float16)kCodeBias, (_Float16)kCodeBias};
  if constexpr (!CLAMP) return y;
  return __builtin_elementwise_min(__builtin_elementwise_max(y, h2_t{(_Float16)(kCodeBias - qmax - 1), (_Float16)(kCodeBias - qmax - 1)}),
                                   h2_t{(_Float16)(kCodeBias + qmax), (_Float16)(kCodeBias + qmax)});
}
// The biased code of x for a zero scale (a group whose max |x| rounds to 0
// in fp16): x / 0 is +-inf (clamped) or NaN for x = 0 (coded 0).
template <int BITS>
__device__ __forceinline__ _Float16 biased_code_zero(float x) {
  constexpr int qmax = (1 << (BITS - 1)) - 1;
  return (_Float16)(kCodeBias + (x > 0.f ? (float)qmax : (x < 0.f ? (float)(-qmax - 1) : 0.f)));
}

// 4-bit residual code of x against the fp32 slot scale s (residual_store.py
// :121-136): clamp(rint(x / s), -8, 7) with x / s rounded to fp32.  The
// Newton quotient q1 is within 1.5 fp32 ulps of the rounded quotient, so the
// two round to the same integer unless q1 lies within 2^-18 of a half
// integer; such lanes take the exact quotient (amb).
__device__ __forceinline__ int res_code(float x, float s, float rc, bool& amb) {
  const float q0 = __builtin_fmaf(x, rc, -0.0f);
  const float e = __builtin_fmaf(-q0, s, x);
  const float q1 = __builtin_fmaf(e, rc, q0);
  const float c = rintf(q1);
  amb = amb || fabsf(q1 - c) > 0.5f - 0x1p-18f;
  return (int)fminf(fmaxf(c, -8.f), 7.f);
}
__device__ __forceinline__ int res_code_exact(float x, float s) {
  return (int)fminf(fmaxf(rintf(x / s), -8.f), 7.f);
}

// Pack 2m fp16 residuals of this lane as 4-bit codes against slot scale s:
// code k at bits 4k (pack_4bit's low nibble first).
template <int NPAIR>
__device__ __forceinline__ uint32_t pack_res(const h2_t* v, float s) {
  const float rc = __builtin_amdgcn_rcpf(s);
  bool amb = false;
  uint32_t w = 0;
#pragma unroll
  for (int p = 0; p < NPAIR; ++p) {
    const int c0 = res_code((float)v[p][0], s, rc, amb), c1 = res_code((float)v[p][1], s, rc, amb);
    w |= (((uint32_t)c0 & 15u) | (((uint32_t)c1 & 15u) << 4)) << (8 * p);
  }
  if (amb) {
    w = 0;
#pragma unroll
    for (int p = 0; p < NPAIR; ++p) {
      const int c0 = res_code_exact((float)v[p][0], s), c1 = res_code_exact((float)v[p][1], s);
      w |= (((uint32_t)c0 & 15u) | (((uint32_t)c1 & 15u) << 4)) << (8 * p);
    }
  }
  return w;
}

// Max |v| over this lane's NPAIR fp16 pairs as fp16 magnitude bits.
template <int NPAIR>
__device__ __forceinline__ uint32_t absmax_bits(const h2_t* v) {
  u16x2_t m = {0, 0};
#pragma unroll
  for (int p = 0; p < NPAIR; ++p)
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, __builtin_bit_cast(uint32_t, v[p]) & 0x7fff7fffu));
  return max((uint32_t)m[0], (uint32_t)m[1]);
}

// Store this lane's W = EPL * BITS code bits F of chunk i.  The page's
// packed rows are one little-endian bit string in which lane l of chunk i
// holds bits [(64 i + l) W, +W); each dword is written whole by one lane.
template <int D, int BITS>
__device__ __forceinline__ void store_code_bits(int8_t* page_rows, int i, int lane, uint32_t F) {
  constexpr int W = (D / 16) * BITS;
  uint32_t* base = reinterpret_cast<uint32_t*>(page_rows) + i * 2 * W;  // chunk i: 64 W bits
  if constexpr (W == 32) {
    base[lane] = F;
  } else if constexpr (W == 16) {
    const uint32_t n = dpp_u<kDppShl1>(F);
    if (!(lane & 1)) base[lane >> 1] = F | (n << 16);
  } else if constexpr (W == 8) {
    const uint32_t a = F | (dpp_u<kDppShl1>(F) << 8);
    const uint32_t b = a | (dpp_u<kDppShl2>(a) << 16);
    if (!(lane & 3)) base[lane >> 2] = b;
  } else if constexpr (W == 24) {  // a quad holds 96 bits = 3 dwords
    const uint32_t n = dpp_u<kDppShl1>(F);
    const int p = lane & 3;
    if (p < 3) base[3 * (lane >> 2) + p] = (F >> (8 * p)) | (n << (24 - 8 * p));
  } else {
    static_assert(W == 12, "code field width");
    const uint32_t G = F | (dpp_u<kDppShl1>(F) << 12);  // lane pairs: 24 bits
    const uint32_t n = dpp_u<kDppShl2>(G);
    const int p = (lane & 7) >> 1;
    if (!(lane & 1) && p < 3) base[3 * (lane >> 3) + p] = (G >> (8 * p)) | (n << (24 - 8 * p));
  }
}
// Read back this lane's W code bits of chunk i (the layout above).
template <int D, int BITS>
__device__ __forceinline__ uint32_t load_code_bits(const int8_t* page_rows, int i, int lane) {
  constexpr int W = (D / 16) * BITS;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(page_rows);
  const int bit = (64 * i + lane) * W;
  const int wi = bit >> 5, sh = bit & 31;
  uint64_t v = w[wi];
  if (sh + W > 32) v |= (uint64_t)w[wi + 1] << 32;
  return (uint32_t)(v >> sh) & (uint32_t)((1ull << W) - 1ull);
}

template <int NP>
__device__ __forceinline__ void load_chunk(uint32_t* w, const uint16_t* p) {
  if constexpr (NP == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  }
}
template <int NP>
__device__ __forceinline__ void store_chunk(uint16_t* p, const uint32_t* w) {
  if constexpr (NP == 4) *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  else *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
}
// EPL int8 codes at p as fp16 pairs.
template <int NP>
__device__ __forceinline__ void load_codes_i8(h2_t* c, const int8_t* p) {
  uint32_t w[(NP + 1) / 2];
  if constexpr (NP == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    const int32_t a = (int32_t)(w[q >> 1] << (24 - 16 * (q & 1))) >> 24;
    const int32_t b = (int32_t)(w[q >> 1] << (16 - 16 * (q & 1))) >> 24;
    c[q] = h2_t{(_Float16)a, (_Float16)b};
  }
}
// Biased fp16 code pairs (1536 + code) -> the W-bit field with code k at
// bits BITS k: the low BITS bits of each half, weighted by dot2.
template <int BITS, int NP>
__device__ __forceinline__ uint32_t code_field(const h2_t* y) {
  constexpr uint32_t M = (1u << BITS) - 1u;
  constexpr int P0 = (15 / BITS - 1) / 2 + 1;  // pairs whose weights fit 16 bits
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const u16x2_t z = __builtin_bit_cast(u16x2_t, __builtin_bit_cast(uint32_t, y[p]) & (M | (M << 16)));
    const int q = p < P0 ? p : p - P0;
    const u16x2_t wgt = {(unsigned short)(1u << (2 * q * BITS)), (unsigned short)(1u << ((2 * q + 1) * BITS))};
    if (p < P0) lo = __builtin_amdgcn_udot2(z, wgt, lo, false);
    else hi = __builtin_amdgcn_udot2(z, wgt, hi, false);
  }
  if constexpr (NP > P0) return lo | (hi << (2 * P0 * BITS));
  else return lo;
}
// The W-bit field -> fp16 code pairs (sign-extended BITS-bit fields).
template <int BITS, int NP>
__device__ __forceinline__ void field_codes(uint32_t F, h2_t* c) {
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int a = (int)(F << (32 - BITS * (2 * p + 1))) >> (32 - BITS);
    const int b = (int)(F << (32 - BITS * (2 * p + 2))) >> (32 - BITS);
    c[p] = h2_t{(_Float16)a, (_Float16)b};
  }
}

// One kind (K or V) of one page: the residual base, the page write
// (codes, scales, master) where the path writes the page, and the
// residual chunks, zero past num_valid.  sq[i]: this lane's partial sum of
// squared residuals of chunk i; vsq: its partial sum of V_hat^2 over the
// valid rows as the decode reads them (V only).
template <int D, int BITS, int PATH, bool IS_V>
__device__ __forceinline__ void store_kind(const carekv_arena& A, const carekv_store_params& sp,
                                           const uint32_t (&x)[4][PageLay<D>::NP], h2_t (&res)[4][PageLay<D>::NP],
                                           float (&sq)[4], float& vsq, StoreLds<D>& S, int lane, long pg,
                                           int job_id, int nvld) {
  using L = PageLay<D>;
  constexpr int EPL = L::EPL, NP = L::NP, LPG = L::LPG, NG = L::NG, P = L::P;
  const int r = lane >> 4, c16 = lane & 15, gl = c16 / LPG, j = c16 % LPG;
  const long tile = (long)job_id * kPage * D;
  const long rows = (long)job_id * kPage;  // first input row of the job
  _Float16 s[4] = {0, 0, 0, 0};            // the rows' group scales (code paths)
  h2_t base[4][NP], code[4][NP];
  uint32_t field[4];                       // packed code bits (page-writing paths)
  _Float16 svr[4] = {0, 0, 0, 0};          // V: scale of V_hat as read back

  if constexpr (PATH == kPathHat || PATH == kPathKivi) {
    const uint16_t* hat = IS_V ? sp.v_hat : sp.k_hat;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t w[NP];
      load_chunk<NP>(w, hat + tile + (long)(4 * i + r) * D + EPL * c16);
#pragma unroll
      for (int p = 0; p < NP; ++p) base[i][p] = __builtin_bit_cast(h2_t, w[p]);
    }
  }
  if constexpr (PATH == kPathFresh) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // max |x| over the group (exact), scale = half(max / qmax)
      const uint32_t m = grp_max_u<LPG>(absmax_bits<NP>(reinterpret_cast<const h2_t*>(x[i])));
      s[i] = group_scale<BITS>(h2f((uint16_t)m));
      const float sf = (float)s[i];
      const float rc = __builtin_amdgcn_rcpf(sf);
      h2_t y[NP];  // 1536 + clamp(rint(half(x / s))) (quantizer.py:58-60)
      if (sf >= 0x1p-14f) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const h2_t xh = __builtin_bit_cast(h2_t, x[i][p]);
          y[p] = biased_codes<BITS, false>(h2_t{quant_q((float)xh[0], sf, rc), quant_q((float)xh[1], sf, rc)});
        }
      } else if (sf != 0.f) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const h2_t xh = __builtin_bit_cast(h2_t, x[i][p]);
          y[p] = biased_codes<BITS, true>(h2_t{quant_q((float)xh[0], sf, rc), quant_q((float)xh[1], sf, rc)});
        }
      } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const h2_t xh = __builtin_bit_cast(h2_t, x[i][p]);
          y[p] = h2_t{biased_code_zero<BITS>((float)xh[0]), biased_code_zero<BITS>((float)xh[1])};
        }
      }
      field[i] = code_field<BITS, NP>(y);
#pragma unroll
      for (int p = 0; p < NP; ++p) code[i][p] = y[p] - h2_t{(_Float16)kCodeBias, (_Float16)kCodeBias};
    }
  } else if constexpr (PATH == kPathKeep) {
    // the page's own base as the decode reads it: half(code * half(scale code * master))
    const int8_t* prow = (IS_V ? A.vcodes : A.kcodes) + pg * kPage * row_bytes(D, BITS);
    const float mst = A.scale_mode == 1 ? h2f((IS_V ? A.vmaster : A.kmaster)[pg]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      field_codes<BITS, NP>(load_code_bits<D, BITS>(prow, i, lane), code[i]);
      const long si = (pg * kPage + 4 * i + r) * NG + gl;
      const void* sc = IS_V ? A.vscale : A.kscale;
      s[i] = A.scale_mode == 1 ? (_Float16)((float)((const int8_t*)sc)[si] * mst)
                               : bits2half(((const uint16_t*)sc)[si]);
      svr[i] = s[i];
    }
  } else if constexpr (PATH == kPathCodesIn || PATH == kPathKivi) {
    const int8_t* cin = IS_V ? sp.v_codes_in : sp.k_codes_in;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      load_codes_i8<NP>(code[i], cin + tile + (long)(4 * i + r) * D + EPL * c16);
      const long ri = (rows + 4 * i + r) * NG + gl;
      if constexpr (PATH == kPathCodesIn) {
        s[i] = bits2half((IS_V ? sp.v_scale_in : sp.k_scale_in)[ri]);
        if (IS_V) {  // V_hat as the page holds it (write_base's scales)
          const long si = (pg * kPage + 4 * i + r) * NG + gl;
          svr[i] = A.scale_mode == 1 ? (_Float16)((float)((const int8_t*)A.vscale)[si] * h2f(A.vmaster[pg]))
                                     : bits2half(((const uint16_t*)A.vscale)[si]);
        }
      } else {
        s[i] = IS_V ? bits2half(sp.v_scale_in[ri]) : (_Float16)0;  // KIVI K: per-channel scales elsewhere
      }
    }
  }

  if constexpr (PATH == kPathFresh || PATH == kPathKivi) {
    // ---- the page: packed codes, scales by (token, group), master
    int8_t* prow = (IS_V ? A.vcodes : A.kcodes) + pg * kPage * row_bytes(D, BITS);
    if constexpr (PATH == kPathKivi) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h2_t y[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) y[p] = code[i][p] + h2_t{(_Float16)kCodeBias, (_Float16)kCodeBias};
        field[i] = code_field<BITS, NP>(y);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) store_code_bits<D, BITS>(prow, i, lane, field[i]);
    if (j == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) S.sf[(4 * i + r) * NG + gl] = half2bits(s[i]);
    }
    lds_sync_wave();
    const int pl = lane % P;
    const _Float16 sp_ = bits2half(S.sf[pl]);
    void* sc = IS_V ? A.vscale : A.kscale;
    if (A.scale_mode == 1) {
      // int8 codes against half(max scale / 127) (cache.py:592-606)
      const float m = h2f((uint16_t)rows_max_u(grp_max_u<16>(half2bits(sp_))));
      const _Float16 mh = (_Float16)(m / 127.f);
      const int8_t q = scale_code((float)sp_, (float)mh);
      if (lane < P) ((int8_t*)sc)[pg * kPage * NG + pl] = q;
      if (lane == 0) (IS_V ? A.vmaster : A.kmaster)[pg] = half2bits(mh);
      if constexpr (IS_V) {
        if (lane < P) S.svr[pl] = half2bits((_Float16)((float)q * (float)mh));
        lds_sync_wave();
#pragma unroll
        for (int i = 0; i < 4; ++i) svr[i] = bits2half(S.svr[(4 * i + r) * NG + gl]);
      }
    } else {
      if (lane < P) ((uint16_t*)sc)[pg * kPage * NG + pl] = half2bits(sp_);
#pragma unroll
      for (int i = 0; i < 4; ++i) svr[i] = s[i];
    }
  }

  // ---- residuals (R = half(X - X_hat), residual_store.py:276-285), zero past num_valid
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t s2 = h2_t{s[i], s[i]};
    float a = 0.f, vs = 0.f;
    const uint32_t keep = 4 * i + r < nvld ? ~0u : 0u;  // rows past num_valid: zero
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const h2_t xh = __builtin_bit_cast(h2_t, x[i][p]);
      h2_t b;
      if constexpr (PATH == kPathHat || PATH == kPathKivi) b = base[i][p];
      else b = code[i][p] * s2;
      const h2_t rr = __builtin_bit_cast(h2_t, __builtin_bit_cast(uint32_t, xh - b) & keep);
      res[i][p] = rr;
      a = __builtin_amdgcn_fdot2(rr, rr, a, false);
      if constexpr (IS_V) {
        h2_t vh;
        if constexpr (PATH == kPathHat) vh = base[i][p];
        else if constexpr (PATH == kPathKeep) vh = b;
        else vh = code[i][p] * h2_t{svr[i], svr[i]};
        vh = __builtin_bit_cast(h2_t, __builtin_bit_cast(uint32_t, vh) & keep);
        vs = __builtin_amdgcn_fdot2(vh, vh, vs, false);
      }
    }
    sq[i] = a;
    if constexpr (IS_V) vsq += vs;
  }

  if constexpr (PATH == kPathHat) {
    // ---- the fp16 side-buffer rows (cache.py:800-818) on the page's code page
    uint16_t* dst = reinterpret_cast<uint16_t*>(IS_V ? A.vcodes : A.kcodes) + code_pg(A, pg) * kPage * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t w[NP];
#pragma unroll
      for (int p = 0; p < NP; ++p) w[p] = __builtin_bit_cast(uint32_t, base[i][p]);
      store_chunk<NP>(dst + (4 * i + r) * D + EPL * c16, w);
    }
  }
}

template <int D, int BITS, int PATH>
__device__ __forceinline__ void store_page(const carekv_arena& A, const carekv_store_params& sp,
                                           const uint16_t* __restrict__ Kx, const uint16_t* __restrict__ Vx,
                                           const carekv_page_job& job, int job_id, StoreWs ws,
                                           const StoreStage& st, StoreLds<D>& S, const float* sP, int SD,
                                           int lane) {
  using L = PageLay<D>;
  constexpr int EPL = L::EPL, NP = L::NP, LPG = L::LPG, NG = L::NG, KSB = L::KSB, VSB = L::VSB;
  const int nvld = job.num_valid;
  const long pg = ((long)job.kv_head * A.n_seq + job.seq) * A.max_pages + job.page;
  // a packed KIVI arena's call runs once over the packed prefix and once
  // over a view of its fp16 tail: each launch takes only its own pages
  if (PATH == kPathKivi && job.page >= A.n_packed[job.seq]) return;
  if (!code_pg_in(A, pg)) return;
  const int r = lane >> 4, c16 = lane & 15, gl = c16 / LPG;
  const long tile = (long)job_id * kPage * D;

  uint32_t xk[4][NP], xv[4][NP];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    load_chunk<NP>(xk[i], Kx + tile + (long)(4 * i + r) * D + EPL * c16);
    load_chunk<NP>(xv[i], Vx + tile + (long)(4 * i + r) * D + EPL * c16);
  }

  // ---- K: page write, residuals, candidate errors, sketch
  h2_t rk[4][NP];
  float sq[4], vsq = 0.f;
  store_kind<D, BITS, PATH, false>(A, sp, xk, rk, sq, vsq, S, lane, pg, job_id, nvld);
  float kn = 0.f;  // sum over this lane's tokens of ||R_K[t, group]||
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float g2 = grp_sum<LPG>(sq[i]);
    kn += 4 * i + r < nvld ? __builtin_amdgcn_sqrtf(g2) : 0.f;
  }
  kn = rows_sum(kn);
  const float kerr_l = nvld > 0 ? kn / (float)nvld : 0.f;  // k_error_norm of group gl
  // residual rows to LDS (the K payloads read them back)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) w[p] = __builtin_bit_cast(uint32_t, rk[i][p]);
    store_chunk<NP>(&S.rk[(4 * i + r) * D + EPL * c16], w);
  }
  // column means of R_K over the valid rows -> sketch half(mean @ P) (residual_store.py:305,311-312)
  {
    float cs[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) a = __builtin_fmaf((float)rk[i][e >> 1][e & 1], 1.0f, a);
      cs[e] = rows_sum(a);
    }
    const float inv = nvld > 0 ? 1.f / (float)nvld : 0.f;
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) S.mean[EPL * c16 + e] = cs[e] * inv;
    }
  }
  lds_sync_wave();
  {
    // sketch[g][k] = sum_c mean[32 g + c] P[c][k] on the fp32 MFMA 16x16x4:
    // A[row = l % 16][kk = l / 16] = mean of channel 4 st + kk of group row (rows
    // past NG zero), B[kk][col] = P[4 st + kk][16 t + col]; lanes 0..15 end with
    // C[row g = 0..3][col = lane] in their four accumulator registers.
    const int T = (SD + 15) >> 4, SDp = 16 * T;
    const int m = lane & 15, kk = lane >> 4;
    float4_t acc[4] = {};
#pragma unroll
    for (int st = 0; st < kGroup / 4; ++st) {
      const float a = m < NG ? S.mean[kGroup * m + 4 * st + kk] : 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (t < T) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, sP[(4 * st + kk) * SDp + 16 * t + m], acc[t], 0, 0, 0);
    }
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t >= T || 16 * t + lane >= SD) continue;
#pragma unroll
        for (int g = 0; g < NG; ++g) A.k_sketch[(pg * NG + g) * SD + 16 * t + lane] = f2h(acc[t][g]);
      }
    }
  }

  // ---- V: page write, residuals, candidate errors, sum of V_hat^2
  h2_t rv[4][NP];
  store_kind<D, BITS, PATH, true>(A, sp, xv, rv, sq, vsq, S, lane, pg, job_id, nvld);
  float verr[kNvb];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float row = grp_sum<16>(sq[i]);
    const float tn = rows_sum(4 * i + r < nvld ? __builtin_amdgcn_sqrtf(row) : 0.f);
    const int cnt = min(max(nvld - 4 * i, 0), kVtb);
    verr[i] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cnt > 0 ? tn / (float)cnt : 0.f)));
  }
  vsq = rows_sum(grp_sum<16>(vsq));

  // ---- uniform candidate errors and the store decision (residual_store.py:372-422).  Every
  // candidate's prior is err * sensitivity * struct_prior with the same positive factor, so
  // priors order as the errors do and are positive where the errors are (sensitivity > 0).
  // The errors are non-negative floats, which order as their bit patterns: the ranks are
  // integer compares of uniform values (a NaN error is not positive, as a NaN prior).
  uint32_t ke[NG], ve[kNvb];
#pragma unroll
  for (int g = 0; g < NG; ++g) ke[g] = (uint32_t)__builtin_amdgcn_readlane(__float_as_int(kerr_l), g * LPG);
#pragma unroll
  for (int b = 0; b < kNvb; ++b) ve[b] = __float_as_uint(verr[b]);
  int nk = 0, nv = 0;
  uint32_t kord = 0, vord = 0;
  if (!sp.store_none && sp.sensitivity > 0.0) {
    bool kp[NG], vp[kNvb];
#pragma unroll
    for (int c = 0; c < NG; ++c) kp[c] = ke[c] - 1u < 0x7f800000u;  // 0 < err <= inf
#pragma unroll
    for (int b = 0; b < kNvb; ++b) vp[b] = ve[b] - 1u < 0x7f800000u;
#pragma unroll
    for (int c = 0; c < NG; ++c) {
      if (!kp[c]) continue;
      int rank = 0, vbefore = 0;  // stable descending order; V before K only on a larger error
#pragma unroll
      for (int c2 = 0; c2 < NG; ++c2) rank += kp[c2] && (ke[c2] > ke[c] || (ke[c2] == ke[c] && c2 < c));
#pragma unroll
      for (int b = 0; b < kNvb; ++b) vbefore += vp[b] && ve[b] > ke[c];
      const bool sel = sp.joint ? rank + vbefore < sp.joint_budget : rank < sp.k_budget;
      if (sel) { kord |= (uint32_t)c << (2 * rank); ++nk; }
    }
#pragma unroll
    for (int b = 0; b < kNvb; ++b) {
      if (!vp[b]) continue;
      int rank = 0, kbefore = 0;
#pragma unroll
      for (int b2 = 0; b2 < kNvb; ++b2) rank += vp[b2] && (ve[b2] > ve[b] || (ve[b2] == ve[b] && b2 < b));
#pragma unroll
      for (int c = 0; c < NG; ++c) kbefore += kp[c] && ke[c] >= ve[b];
      const bool sel = sp.joint ? rank + kbefore < sp.joint_budget : rank < sp.v_budget;
      if (sel) { vord |= (uint32_t)b << (2 * rank); ++nv; }
    }
  }

  // ---- payloads of the selections, in slot order, to the staging area
  const int ms = st.mk + st.mv;
  for (int i = 0; i < nk; ++i) {
    const int c = (kord >> (2 * i)) & 3;
    // pack_4bit(R_K[:, cg]): lane l takes token l / 4, channels 8 (l % 4) .. + 7 of the group
    const uint4 raw = *reinterpret_cast<const uint4*>(&S.rk[(lane >> 2) * D + kGroup * c + 8 * (lane & 3)]);
    const h2_t v[4] = {__builtin_bit_cast(h2_t, raw.x), __builtin_bit_cast(h2_t, raw.y),
                       __builtin_bit_cast(h2_t, raw.z), __builtin_bit_cast(h2_t, raw.w)};
    const float m = h2f((uint16_t)rows_max_u(grp_max_u<16>(absmax_bits<4>(v))));
    const float s = fmaxf(m, 1e-8f) / 7.0f;
    const uint32_t w = pack_res<4>(v, s);
    *reinterpret_cast<uint32_t*>(st.kpay + ((long)job_id * st.mk + i) * KSB + 4 * lane) = w;
    if (lane == 0) st.scale[(long)job_id * ms + i] = f2h(s);
  }
  for (int i = 0; i < nv; ++i) {
    const int b = (vord >> (2 * i)) & 3;
    // pack_4bit(R_V[4b .. 4b+3, :]): chunk b of every lane, in row-major order
    h2_t v[NP];
    switch (b) {  // b is uniform
      case 0: for (int p = 0; p < NP; ++p) v[p] = rv[0][p]; break;
      case 1: for (int p = 0; p < NP; ++p) v[p] = rv[1][p]; break;
      case 2: for (int p = 0; p < NP; ++p) v[p] = rv[2][p]; break;
      default: for (int p = 0; p < NP; ++p) v[p] = rv[3][p]; break;
    }
    const float m = h2f((uint16_t)rows_max_u(grp_max_u<16>(absmax_bits<NP>(v))));
    const float s = fmaxf(m, 1e-8f) / 7.0f;
    const uint32_t w = pack_res<NP>(v, s);
    int8_t* dst = st.vpay + ((long)job_id * st.mv + i) * VSB + (EPL / 2) * lane;
    if constexpr (NP == 4) *reinterpret_cast<uint32_t*>(dst) = w;
    else *reinterpret_cast<uint16_t*>(dst) = (uint16_t)w;
    if (lane == 0) st.scale[(long)job_id * ms + st.mk + i] = f2h(s);
  }

  // ---- metadata, counts (the streaming fill store reuses the page's earlier ids first)
  if (lane < NG * LPG && (lane & (LPG - 1)) == 0) A.k_err[pg * NG + gl] = f2h(kerr_l);
  if (lane < kNvb) A.v_err[pg * kNvb + lane] = f2h(lane == 0 ? verr[0] : (lane == 1 ? verr[1] : (lane == 2 ? verr[2] : verr[3])));
  if (lane == 0) {
    int n_ok = 0, n_ov = 0;
    if (sp.reuse_slots && A.has_meta[pg]) {
#pragma unroll
      for (int c = 0; c < NG; ++c) n_ok += A.k_slot[pg * NG + c] >= 0;
#pragma unroll
      for (int b = 0; b < kNvb; ++b) n_ov += A.v_slot[pg * kNvb + b] >= 0;
    }
    A.v_sq[pg] = vsq;
    st.head[job_id] = (uint32_t)nk | ((uint32_t)nv << 3) | ((uint32_t)n_ok << 6) | ((uint32_t)n_ov << 9) |
                      (kord << 12) | (vord << 20);
    ws.v[job_id * 4 + 0] = nk - min(n_ok, nk);
    ws.v[job_id * 4 + 1] = nv - min(n_ov, nv);
  }
}

// Page jobs of a store call: an explicit job array with its sequence
// groups, or a prompt chunk's grid (carekv_prefill_grid) that generates
// job j = (row b, kv head h, page p) in row-major order, group b = row b.
struct JobSrc {
  const carekv_page_job* jobs;  // nullptr: the grid
  const int32_t* group_ptr;
  const int32_t* rows;          // grid: row slots, then first page ids
  int32_t n_rows, n_kvh, n_pages, n_tokens, token_start;
  __device__ __forceinline__ carekv_page_job get(int j) const {
    if (jobs) return jobs[j];
    const int p = j % n_pages, bh = j / n_pages, b = bh / n_kvh, h = bh - b * n_kvh;
    carekv_page_job o;
    o.seq = rows[b];
    o.kv_head = h;
    o.page = rows[n_rows + bh] + p;
    o.num_valid = min(kPage, n_tokens - kPage * p);
    o.token_start = token_start + kPage * p;
    o.is_recent = p >= n_pages - 4;
    return o;
  }
  __device__ __forceinline__ void group(int g, int& j0, int& j1) const {
    if (jobs) {
      j0 = group_ptr[g];
      j1 = group_ptr[g + 1];
    } else {
      j0 = g * n_kvh * n_pages;
      j1 = j0 + n_kvh * n_pages;
    }
  }
};

// Bytes of the sketch projection at the start of the store pass's LDS: the
// 32 x sketch_dim fp32 matrix with its rows padded to a multiple of 16.
__host__ __device__ constexpr int store_lds_p_bytes(int sd) { return kGroup * ((sd + 15) / 16 * 16) * 4; }

// The store pass: each wave takes jobs blockIdx.x * 4 + wave, then every
// gridDim.x * 4-th; the sketch projection sits in LDS for the whole block.
template <int D, int BITS, int PATH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 && PATH != kPathKivi ? 4 : 1))) void store_pages_kernel(carekv_arena A, carekv_store_params sp,
                                                          const uint16_t* __restrict__ Kx,
                                                          const uint16_t* __restrict__ Vx, JobSrc src,
                                                          int n_jobs, StoreWs ws, StoreStage st) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int SD = A.sketch_dim, SDp = (SD + 15) / 16 * 16;
  float* sP = reinterpret_cast<float*>(smem);
  for (int k = threadIdx.x; k < kGroup * SDp; k += 256) {
    const int c = k / SDp, n = k - c * SDp;
    sP[k] = n < SD ? sp.sketch_proj[c * SD + n] : 0.f;
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  StoreLds<D>& S = reinterpret_cast<StoreLds<D>*>(smem + store_lds_p_bytes(SD))[wave];
  // the call's slot-overflow word (after the job records) starts clear; the scatter sets it
  if (blockIdx.x == 0 && threadIdx.x == 0) ws.v[n_jobs * 4] = 0;
  for (int job_id = blockIdx.x * 4 + wave; job_id < n_jobs; job_id += gridDim.x * 4)
    store_page<D, BITS, PATH>(A, sp, Kx, Vx, src.get(job_id), job_id, ws, st, S, sP, SD, lane);
}

// Exclusive scan of the per-job new-slot counts inside each sequence group
// (jobs of one group are contiguous and ordered like the reference's
// process_page calls); bases start at next_slot[seq], which is advanced.
// One block of 1024 threads per group.  A round takes up to kScanRows rows
// of 1024 jobs; thread t holds job 1024 k + t of every row k, so loads and
// stores are lane-consecutive and all of a round's loads are in flight at
// once.  A job's base is the carry, plus the totals of the rows before
// its own, plus the totals of the waves before its own in its row, plus
// the wave-level exclusive scan.  Counts are at most 4 per job, so a wave
// scans K and V counts packed as K | V << 16.
constexpr int kScanRows = 24;
__global__ __launch_bounds__(1024) void store_scan_kernel(carekv_arena A, JobSrc src, StoreWs ws) {
  __shared__ uint32_t s_wave[kScanRows][16];  // per row and wave: total (packed), then exclusive prefix
  __shared__ int2 s_row[kScanRows];           // per row: exclusive prefix over the rows (K, V)
  __shared__ int2 s_tot;
  const int g = blockIdx.x;
  int j0, j1;
  src.group(g, j0, j1);
  if (j1 <= j0) return;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int n = j1 - j0;
  const int seq = src.get(j0).seq;
  int carry_k = A.next_slot[2 * seq], carry_v = A.next_slot[2 * seq + 1];
  for (int base = 0; base < n; base += 1024 * kScanRows) {
    const int rows = min(kScanRows, (n - base + 1023) / 1024);
    uint32_t c[kScanRows], inc[kScanRows];
#pragma unroll
    for (int k = 0; k < kScanRows; ++k) {
      const int j = base + 1024 * k + t;
      c[k] = 0;
      if (k < rows && j < n) {
        const int2 v = *reinterpret_cast<const int2*>(ws.v + (long)(j0 + j) * 4);
        c[k] = (uint32_t)v.x | ((uint32_t)v.y << 16);
      }
    }
#pragma unroll
    for (int k = 0; k < kScanRows; ++k) {
      if (k >= rows) break;
      uint32_t x = c[k];  // inclusive scan over the wave
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
      }
      inc[k] = x;
      if (lane == 63) s_wave[k][w] = x;
    }
    __syncthreads();
    if (t < rows * 16) {  // one thread per (row, wave): exclusive prefix over the row's waves
      // (the 16 threads of a row are one quarter of one wave: all its reads precede its writes)
      const int k = t >> 4, ww = t & 15;
      uint32_t pre = 0, tot = 0;
      for (int i = 0; i < 16; ++i) {
        const uint32_t v = s_wave[k][i];
        pre += i < ww ? v : 0u;
        tot += v;
      }
      s_wave[k][ww] = pre;
      if (ww == 0) s_row[k] = make_int2((int)(tot & 0xffffu), (int)(tot >> 16));
    }
    __syncthreads();
    if (t == 0) {  // exclusive prefix over the rows
      int pk = 0, pv = 0;
      for (int k = 0; k < rows; ++k) {
        const int2 v = s_row[k];
        s_row[k] = make_int2(pk, pv);
        pk += v.x;
        pv += v.y;
      }
      s_tot = make_int2(pk, pv);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kScanRows; ++k) {
      if (k >= rows) break;
      const int j = base + 1024 * k + t;
      const uint32_t ex = s_wave[k][w] + inc[k] - c[k];  // packed, per field < 2^16
      const int2 r = s_row[k];
      if (j < n)
        *reinterpret_cast<int2*>(ws.v + (long)(j0 + j) * 4 + 2) =
            make_int2(carry_k + r.x + (int)(ex & 0xffffu), carry_v + r.y + (int)(ex >> 16));
    }
    carry_k += s_tot.x;
    carry_v += s_tot.y;
    __syncthreads();  // LDS is rewritten by the next round
  }
  if (t == 0) { A.next_slot[2 * seq] = carry_k; A.next_slot[2 * seq + 1] = carry_v; }
}

// Slot id of the i-th selection of a kind: the page's earlier ids first
// (ascending), then new ids from the scanned base; -1 past the arena.
__device__ __forceinline__ int slot_of(int i, int n_old, const int* old, int n_cand, int base, int n_slots) {
  if (i < n_old) {
    // the i-th smallest of the page's earlier ids (>= 0), n_cand entries
    int id = -1;
#pragma unroll
    for (int c = 0; c < n_cand; ++c) {
      if (old[c] < 0) continue;
      int rank = 0;
#pragma unroll
      for (int c2 = 0; c2 < n_cand; ++c2) rank += old[c2] >= 0 && old[c2] < old[c];
      if (rank == i) id = old[c];
    }
    return id;
  }
  const int id = base + (i - n_old);
  return id < n_slots ? id : -1;
}

// The scatter: slot tables, slot payloads and scales, valid / has_meta of
// every job (residual_store.py:424-438).  16 lanes per job, 16 jobs a block.
template <int D>
__global__ __launch_bounds__(256) void store_slots_kernel(carekv_arena A, JobSrc src, int n_jobs, StoreWs ws,
                                                          StoreStage st) {
  using L = PageLay<D>;
  constexpr int NG = L::NG, KSB = L::KSB, VSB = L::VSB, VP = VSB / 16;
  const int sub = threadIdx.x & 15;
  const int job_id = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (job_id >= n_jobs) return;
  const carekv_page_job job = src.get(job_id);
  const uint32_t h = st.head[job_id];
  const int2 base = *reinterpret_cast<const int2*>(ws.v + (long)job_id * 4 + 2);
  const long pg = ((long)job.kv_head * A.n_seq + job.seq) * A.max_pages + job.page;
  const int nk = min((int)(h & 7), st.mk), nv = min((int)((h >> 3) & 7), st.mv);
  const int n_ok = (h >> 6) & 7, n_ov = (h >> 9) & 7;
  int old_k[NG], old_v[kNvb];
#pragma unroll
  for (int c = 0; c < NG; ++c) old_k[c] = n_ok ? A.k_slot[pg * NG + c] : -1;
#pragma unroll
  for (int b = 0; b < kNvb; ++b) old_v[b] = n_ov ? A.v_slot[pg * kNvb + b] : -1;
  const long seq_off = (long)job.seq * A.n_slots;
  const int ms = st.mk + st.mv;
  // payloads: lane sub copies 16-byte piece sub of each
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    if (i >= nk) break;
    const int id = slot_of(i, n_ok, old_k, NG, base.x, A.n_slots);
    const uint4 v = *reinterpret_cast<const uint4*>(st.kpay + ((long)job_id * st.mk + i) * KSB + 16 * sub);
    if (id >= 0) *reinterpret_cast<uint4*>(A.k_res + (seq_off + id) * KSB + 16 * sub) = v;
  }
#pragma unroll
  for (int i = 0; i < kNvb; ++i) {
    if (i >= nv) break;
    if (sub < VP) {
      const int id = slot_of(i, n_ov, old_v, kNvb, base.y, A.n_slots);
      const uint4 v = *reinterpret_cast<const uint4*>(st.vpay + ((long)job_id * st.mv + i) * VSB + 16 * sub);
      if (id >= 0) *reinterpret_cast<uint4*>(A.v_res + (seq_off + id) * VSB + 16 * sub) = v;
    }
  }
  if (sub < NG) {  // slot tables: candidate c holds the id of its selection, -1 if none
    int id = -1;
    for (int i = 0; i < nk; ++i)
      if ((int)((h >> (12 + 2 * i)) & 3) == sub) id = slot_of(i, n_ok, old_k, NG, base.x, A.n_slots);
    A.k_slot[pg * NG + sub] = id;
  } else if (sub >= 4 && sub < 4 + nk) {
    const int id = slot_of(sub - 4, n_ok, old_k, NG, base.x, A.n_slots);
    if (id >= 0) A.k_res_scale[seq_off + id] = st.scale[(long)job_id * ms + sub - 4];
  } else if (sub >= 8 && sub < 8 + kNvb) {
    const int b = sub - 8;
    int id = -1;
    for (int i = 0; i < nv; ++i)
      if ((int)((h >> (20 + 2 * i)) & 3) == b) id = slot_of(i, n_ov, old_v, kNvb, base.y, A.n_slots);
    A.v_slot[pg * kNvb + b] = id;
  } else if (sub >= 12 && sub < 12 + nv) {
    const int id = slot_of(sub - 12, n_ov, old_v, kNvb, base.y, A.n_slots);
    if (id >= 0) A.v_res_scale[seq_off + id] = st.scale[(long)job_id * ms + st.mk + sub - 12];
  }
  if (sub == 15) {
    A.valid[pg] = job.num_valid;
    A.has_meta[pg] = 1;
    // new ids past the arena are dropped (never written) and flagged
    if ((nk > n_ok && base.x + (nk - n_ok) > A.n_slots) || (nv > n_ov && base.y + (nv - n_ov) > A.n_slots))
      ws.v[n_jobs * 4] = 1;
  }
}

// KIVI-style value (kivi_helpers.py:35-59): half(clamp(rint(half(x / s))) * s)
// in fp16 arithmetic; a NaN quotient (0/0) stays NaN through rint and
// clamp, as torch's clamp propagates it.
__device__ __forceinline__ float kivi_value(float x, float scale, int bits) {
  const float qmax = (float)((1 << (bits - 1)) - 1);
  const float q = rintf((float)(_Float16)(x / scale));
  const float c = (q != q) ? q : fminf(fmaxf(q, -qmax - 1.f), qmax);
  // the product's sign is the code's (scale >= 0): a code of -0 (the rint of
  // a small negative quotient) gives -0 as in the reference, which a fused
  // multiply-add with a +0 addend would turn into +0
  const float r = (float)(_Float16)(c * scale);
  return (c != c) ? r : copysignf(r, c);
}
// scale = half(max|x| / qmax); the 1e-8 floor is 0 in fp16 (a no-op)
__device__ __forceinline__ float kivi_scale(float amax, int bits) {
  return (float)(_Float16)(amax / (float)((1 << (bits - 1)) - 1));
}

// quant_dequant_kivi_k: one work-group per (matrix, 64 columns); 4 row
// groups reduce max|x| per column through LDS.
__global__ __launch_bounds__(256) void kivi_channel_kernel(const uint16_t* __restrict__ x, int rows, int D, int bits,
                                                           uint16_t* __restrict__ out) {
  __shared__ float s_max[4][64];
  const int m = blockIdx.x, c0 = blockIdx.y * 64;
  const int lane = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int d = c0 + lane;
  const long base = (long)m * rows * D;
  float a = 0.f;
  if (d < D)
    for (int r = rg; r < rows; r += 4) a = fmaxf(a, fabsf(h2f(x[base + (long)r * D + d])));
  s_max[rg][lane] = a;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_max[0][lane], s_max[1][lane]), fmaxf(s_max[2][lane], s_max[3][lane]));
  const float sc = kivi_scale(amax, bits);
  if (d < D)
    for (int r = rg; r < rows; r += 4) {
      const long i = base + (long)r * D + d;
      out[i] = f2h(kivi_value(h2f(x[i]), sc, bits));
    }
}

// quant_dequant_kivi_v: one wave per row.
__global__ __launch_bounds__(256) void kivi_token_kernel(const uint16_t* __restrict__ x, long n_rows, int D, int bits,
                                                         uint16_t* __restrict__ out) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;
  const uint16_t* xr = x + row * D;
  float a = 0.f;
  for (int d = lane; d < D; d += 64) a = fmaxf(a, fabsf(h2f(xr[d])));
  const float sc = kivi_scale(wave_max(a), bits);
  for (int d = lane; d < D; d += 64) out[row * D + d] = f2h(kivi_value(h2f(xr[d]), sc, bits));
}

// Decode append for the fp16 side-buffer base: one wave per row; K per
// channel over the one row (scale |k_d| / qmax), V per token
// (layer.py:1037-1075, cache.py:820-838).
template <int D>
__global__ __launch_bounds__(256) void append_hat_rows_kernel(carekv_arena A, const uint16_t* __restrict__ Kx,
                                                              const uint16_t* __restrict__ Vx,
                                                              const int32_t* __restrict__ dest, int n_rows) {
  constexpr int NG = D / 32;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int seq = dest[row * 4], kvh = dest[row * 4 + 1], page = dest[row * 4 + 2], fresh = dest[row * 4 + 3];
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int off = fresh ? 0 : A.valid[pg];
  if (off >= kPage) return;  // caller contract violated; never write past the page
  if (!code_pg_in(A, pg)) return;  // a page the code-page map does not hold: never written
  const long cpg = code_pg(A, pg);
  uint16_t* krow = reinterpret_cast<uint16_t*>(A.kcodes) + (cpg * kPage + off) * D;
  uint16_t* vrow = reinterpret_cast<uint16_t*>(A.vcodes) + (cpg * kPage + off) * D;
  float av = 0.f;
  for (int d = lane; d < D; d += 64) av = fmaxf(av, fabsf(h2f(Vx[(long)row * D + d])));
  const float sv = kivi_scale(wave_max(av), A.hat_bits_v);
  float vs = 0.f;  // this row's share of the page's sum of V_hat^2
  for (int d = lane; d < D; d += 64) {
    const float k = h2f(Kx[(long)row * D + d]);
    krow[d] = f2h(kivi_value(k, kivi_scale(fabsf(k), A.hat_bits_k), A.hat_bits_k));
    const uint16_t vh = f2h(kivi_value(h2f(Vx[(long)row * D + d]), sv, A.hat_bits_v));
    vrow[d] = vh;
    vs += h2f(vh) * h2f(vh);
  }
  vs = wave_sum(vs);
  // the store on fill, unless the caller's streaming store writes the page's
  // metadata (it reads the slots the page holds)
  const bool full = off + 1 == kPage && !A.streaming_store;
  if (lane == 0) {
    A.valid[pg] = off + 1;
    if (fresh) A.has_meta[pg] = full ? 1 : 0;
    if (full) A.has_meta[pg] = 1;
    A.v_sq[pg] = full ? 0.f : (fresh ? 0.f : A.v_sq[pg]) + vs;
  }
  if (full) {
    // store on page fill with K_orig = K_hat: zero residual -> no slots,
    // zero errors, zero sketch (layer.py:1088-1101)
    if (lane < NG) { A.k_slot[pg * NG + lane] = -1; A.k_err[pg * NG + lane] = 0; }
    if (lane < kVtb) { A.v_slot[pg * kVtb + lane] = -1; A.v_err[pg * kVtb + lane] = 0; }
    for (int i = lane; i < NG * A.sketch_dim; i += 64) A.k_sketch[pg * NG * A.sketch_dim + i] = 0;
  }
}

// Decode append: one wave per (row); lane g < D/32 quantizes group g.
// Int8 page scales (scale_mode 1) take one of two encodings:
//   * the reference's (cache.py:689-695): the row's scale codes against the
//     page's fixed master, clamped at 1e-8 -- a page the decode opens keeps
//     master 0, so its rows read back as zero;
//   * rescale_open: the page is encoded as write_base encodes a page holding
//     its valid rows (cache.py:592-604): master = half(max scale / 127) over
//     the rows so far and every row's code against it, from the fp16 scales
//     of the open page kept in open_kscale / open_vscale (this row's are
//     added there).  When the page fills, its bytes are those write_base
//     gives the 16 rows.  A page that holds stored residual slots (a
//     prompt's partial last page) is not re-encoded: its slots are residuals
//     against its rows as the prompt wrote them, so it keeps the reference's
//     fixed-master encoding (the first form) until it fills.
// The page's sum of V_hat^2 (v_sq, read by the query-aware K score of its
// stored K slots) is recomputed over the valid rows as they now read back.
// Coded rows (append_to_page, cache.py:656-701): the caller's int8 codes and
// fp16 group scales replace the row quantizer, and a full page gets no
// metadata (the store on fill belongs to the decode step, not the append).
struct CodedRows {
  const int8_t* kc;
  const uint16_t* ks;
  const int8_t* vc;
  const uint16_t* vs;
};

template <int D, int BITS>
__global__ __launch_bounds__(256) void append_rows_kernel(carekv_arena A, const uint16_t* __restrict__ Kx,
                                                          const uint16_t* __restrict__ Vx,
                                                          const int32_t* __restrict__ dest, int n_rows,
                                                          CodedRows cr) {
  constexpr int NG = D / 32;
  constexpr int RB = row_bytes(D, BITS);
  constexpr int CB = 4 * BITS;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int seq = dest[row * 4], kvh = dest[row * 4 + 1], page = dest[row * 4 + 2], fresh = dest[row * 4 + 3];
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int off = fresh ? 0 : A.valid[pg];
  if (off >= kPage) return;  // caller contract violated; never write past the page
  const bool i8 = A.scale_mode == 1;
  // stored slots on the page (only a page with metadata can hold any)
  bool slots = false;
  if (!fresh && A.has_meta[pg]) {
    const int id = lane < NG ? A.k_slot[pg * NG + lane]
                             : (lane < NG + kVtb ? A.v_slot[pg * kVtb + lane - NG] : -1);
    slots = __ballot(id >= 0) != 0ull;
  }
  const bool rescale = i8 && A.rescale_open != 0 && !slots;
  int cv[32];
  _Float16 sk = (_Float16)0.f, sv = (_Float16)0.f;
  if (lane < NG) {
    const int g = lane;
    float xk[32], xv[32];
    int ck[32];
    if (cr.kc) {
      for (int i = 0; i < 32; ++i) {
        ck[i] = cr.kc[(long)row * D + g * 32 + i];
        cv[i] = cr.vc[(long)row * D + g * 32 + i];
      }
      sk = bits2half(cr.ks[(long)row * NG + g]);
      sv = bits2half(cr.vs[(long)row * NG + g]);
    } else {
      for (int i = 0; i < 32; ++i) {
        xk[i] = h2f(Kx[(long)row * D + g * 32 + i]);
        xv[i] = h2f(Vx[(long)row * D + g * 32 + i]);
      }
      sk = quant_group<BITS>(xk, ck);
      sv = quant_group<BITS>(xv, cv);
    }
    uint32_t w[BITS];
    pack_group<BITS>(ck, w);
    store_bytes<CB>(A.kcodes + (pg * kPage + off) * RB + g * CB, w);
    pack_group<BITS>(cv, w);
    store_bytes<CB>(A.vcodes + (pg * kPage + off) * RB + g * CB, w);
    if (!i8) {
      ((uint16_t*)A.kscale)[(pg * kPage + off) * NG + g] = half2bits(sk);
      ((uint16_t*)A.vscale)[(pg * kPage + off) * NG + g] = half2bits(sv);
    }
  }
  // lane l < 16 NG: row r = l / NG, group gg = l % NG of the page
  const int r = lane / NG, gg = lane % NG;
  const bool cell = lane < kPage * NG && r <= off;
  float mk = 0.f, mv = 0.f;  // the page's masters after this row (int8 scales)
  if (rescale) {
    const long ob = ((long)kvh * A.n_seq + seq) * kPage * NG;
    const float nk = __shfl((float)sk, gg, 64), nv = __shfl((float)sv, gg, 64);
    float s_k = 0.f, s_v = 0.f;
    if (cell) {
      s_k = r < off ? h2f(A.open_kscale[ob + r * NG + gg]) : nk;
      s_v = r < off ? h2f(A.open_vscale[ob + r * NG + gg]) : nv;
    }
    mk = (float)(_Float16)(wave_max(s_k) / 127.f);
    mv = (float)(_Float16)(wave_max(s_v) / 127.f);
    if (cell) {
      ((int8_t*)A.kscale)[(pg * kPage + r) * NG + gg] = scale_code(s_k, mk);
      ((int8_t*)A.vscale)[(pg * kPage + r) * NG + gg] = scale_code(s_v, mv);
    }
    if (lane < NG) {
      A.open_kscale[ob + off * NG + lane] = half2bits(sk);
      A.open_vscale[ob + off * NG + lane] = half2bits(sv);
    }
  } else if (i8) {
    mk = fmaxf(fresh ? 0.f : h2f(A.kmaster[pg]), 1e-8f);
    mv = fmaxf(fresh ? 0.f : h2f(A.vmaster[pg]), 1e-8f);
    if (lane < NG) {
      ((int8_t*)A.kscale)[(pg * kPage + off) * NG + lane] = scale_code((float)sk, mk);
      ((int8_t*)A.vscale)[(pg * kPage + off) * NG + lane] = scale_code((float)sv, mv);
    }
  }
  // sum of V_hat^2 over the valid rows: earlier rows from the page, this row
  // from the registers of lanes g < NG
  float vs = 0.f;
  if (lane < NG) {
    _Float16 s = sv;
    if (i8) s = (_Float16)((float)scale_code((float)sv, mv) * (rescale ? mv : (fresh ? 0.f : h2f(A.vmaster[pg]))));
#pragma unroll
    for (int i = 0; i < 32; ++i) { const float x = (float)dq(cv[i], s); vs += x * x; }
  }
  if (cell && r < off) {
    uint32_t w[BITS];
    load_bytes<CB>(w, A.vcodes + (pg * kPage + r) * RB + gg * CB);
    _Float16 s;
    if (i8) {
      const int8_t q = ((const int8_t*)A.vscale)[(pg * kPage + r) * NG + gg];
      s = (_Float16)((float)(rescale ? scale_code(h2f(A.open_vscale[((long)kvh * A.n_seq + seq) * kPage * NG +
                                                                    r * NG + gg]), mv) : q) *
                     (rescale ? mv : h2f(A.vmaster[pg])));
    } else {
      s = bits2half(((const uint16_t*)A.vscale)[(pg * kPage + r) * NG + gg]);
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) { const float x = (float)dq(get_code<BITS>(w, i), s); vs += x * x; }
  }
  vs = wave_sum(vs);
  // the decode step's store on fill, unless the caller's streaming store
  // writes the page's metadata (it reads the slots the page holds)
  const bool full = off + 1 == kPage && !cr.kc && !A.streaming_store;
  if (lane == 0) {
    A.valid[pg] = off + 1;
    if (rescale) { A.kmaster[pg] = half2bits((_Float16)mk); A.vmaster[pg] = half2bits((_Float16)mv); }
    else if (fresh && i8) { A.kmaster[pg] = 0; A.vmaster[pg] = 0; }
    if (fresh) A.has_meta[pg] = full ? 1 : 0;
    if (full) A.has_meta[pg] = 1;
    A.v_sq[pg] = full ? 0.f : vs;
  }
  if (full) {
    // store on page fill with K_orig = K_hat: zero residual -> no slots,
    // zero errors, zero sketch (layer.py:1088-1146)
    if (lane < NG) { A.k_slot[pg * NG + lane] = -1; A.k_err[pg * NG + lane] = 0; }
    if (lane < kVtb) { A.v_slot[pg * kVtb + lane] = -1; A.v_err[pg * kVtb + lane] = 0; }
    for (int i = lane; i < NG * A.sketch_dim; i += 64) A.k_sketch[pg * NG * A.sketch_dim + i] = 0;
  }
}

// read_base_concat for one (seq, kv head): unpacked codes + fp16 scales.
template <int D, int BITS>
__global__ __launch_bounds__(256) void read_pages_kernel(carekv_arena A, int seq, int kvh, int n_pages,
                                                         const int32_t* __restrict__ page_ids,
                                                         const int32_t* __restrict__ row_start, int8_t* kc,
                                                         uint16_t* ks, int8_t* vc, uint16_t* vs) {
  constexpr int NG = D / 32;
  constexpr int RB = row_bytes(D, BITS);
  constexpr int CB = 4 * BITS;
  const int p = blockIdx.x;
  if (p >= n_pages) return;
  const int page = page_ids ? page_ids[p] : p;
  if (page < 0 || page >= A.max_pages) return;
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int n = A.valid[pg];
  const int r0 = row_start[p];
  for (int idx = threadIdx.x; idx < n * NG; idx += blockDim.x) {
    const int t = idx / NG, g = idx % NG;
    const long out_row = r0 + t;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      const int8_t* src = (which ? A.vcodes : A.kcodes) + (pg * kPage + t) * RB + g * CB;
      uint32_t w[BITS];
      load_bytes<CB>(w, src);
      int8_t* dst = (which ? vc : kc) + out_row * D + g * 32;
      for (int i = 0; i < 32; ++i) dst[i] = (int8_t)get_code<BITS>(w, i);
      uint16_t s;
      if (A.scale_mode == 1) {
        const int8_t q = ((const int8_t*)(which ? A.vscale : A.kscale))[(pg * kPage + t) * NG + g];
        const uint16_t m = which ? A.vmaster[pg] : A.kmaster[pg];
        s = f2h((float)q * h2f(m));
      } else {
        s = ((const uint16_t*)(which ? A.vscale : A.kscale))[(pg * kPage + t) * NG + g];
      }
      (which ? vs : ks)[out_row * NG + g] = s;
    }
  }
}

// Codes and scales of the KIVI quant-dequant (carekv_kivi_codes): one
// work-group per (matrix, 64 columns) for K per channel over the rows, one
// wave per row for V per token.  A scale whose max|x| is 0 is stored as NaN.
__device__ __forceinline__ int kivi_code(float x, float scale, int bits) {
  const float qmax = (float)((1 << (bits - 1)) - 1);
  const float q = rintf((float)(_Float16)(x / scale));
  return (q != q) ? 0 : (int)fminf(fmaxf(q, -qmax - 1.f), qmax);
}
__global__ __launch_bounds__(256) void kivi_channel_codes_kernel(const uint16_t* __restrict__ x, int rows, int D,
                                                                 int bits, int8_t* __restrict__ codes,
                                                                 uint16_t* __restrict__ scale) {
  __shared__ float s_max[4][64];
  const int m = blockIdx.x, c0 = blockIdx.y * 64;
  const int lane = threadIdx.x & 63, rg = threadIdx.x >> 6;
  const int d = c0 + lane;
  const long base = (long)m * rows * D;
  float a = 0.f;
  if (d < D)
    for (int r = rg; r < rows; r += 4) a = fmaxf(a, fabsf(h2f(x[base + (long)r * D + d])));
  s_max[rg][lane] = a;
  __syncthreads();
  const float amax = fmaxf(fmaxf(s_max[0][lane], s_max[1][lane]), fmaxf(s_max[2][lane], s_max[3][lane]));
  const float sc = kivi_scale(amax, bits);
  if (d < D) {
    for (int r = rg; r < rows; r += 4) {
      const long i = base + (long)r * D + d;
      codes[i] = (int8_t)kivi_code(h2f(x[i]), sc, bits);
    }
    if (rg == 0) scale[(long)m * D + d] = amax == 0.f ? (uint16_t)0x7e00u : f2h(sc);
  }
}
__global__ __launch_bounds__(256) void kivi_token_codes_kernel(const uint16_t* __restrict__ x, long n_rows, int D,
                                                               int bits, int8_t* __restrict__ codes,
                                                               uint16_t* __restrict__ scale) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;
  const uint16_t* xr = x + row * D;
  float a = 0.f;
  for (int d = lane; d < D; d += 64) a = fmaxf(a, fabsf(h2f(xr[d])));
  const float amax = wave_max(a);
  const float sc = kivi_scale(amax, bits);
  for (int d = lane; d < D; d += 64) codes[row * D + d] = (int8_t)kivi_code(h2f(xr[d]), sc, bits);
  if (lane == 0) scale[row] = amax == 0.f ? (uint16_t)0x7e00u : f2h(sc);
}

// read_base_hat_concat (carekv_read_hat_pages): one 64-thread block per page;
// K_hat / V_hat rows of a fp16 page (the side-buffer base, or the tail of a
// packed KIVI arena) copied, of a packed KIVI prefix page dequantised.
template <int D>
__global__ __launch_bounds__(64) void read_hat_pages_kernel(carekv_arena A, int seq, int kvh, int n_pages,
                                                            const int32_t* __restrict__ page_ids,
                                                            const int32_t* __restrict__ row_start,
                                                            uint16_t* __restrict__ kh, uint16_t* __restrict__ vh) {
  constexpr int NG = D / 32;
  constexpr int RB2 = row_bytes(D, 2);
  const int p = blockIdx.x;
  if (p >= n_pages) return;
  const int page = page_ids ? page_ids[p] : p;
  if (page < 0 || page >= A.max_pages) return;
  const long pg = ((long)kvh * A.n_seq + seq) * A.max_pages + page;
  const int n = A.valid[pg];
  const long r0 = row_start[p];
  const bool packed = A.kivi_packed && page < A.n_packed[seq];
  if (packed) {
    const uint16_t* kc = A.kchan + ((long)kvh * A.n_seq + seq) * D;
    for (int idx = threadIdx.x; idx < n * D; idx += 64) {
      const int t = idx / D, d = idx % D, g = d / 32;
      uint32_t w[2];
      load_bytes<8>(w, A.kcodes + (pg * kPage + t) * RB2 + g * 8);
      const int ck = get_code<2>(w, d % 32);
      load_bytes<8>(w, A.vcodes + (pg * kPage + t) * RB2 + g * 8);
      const int cv = get_code<2>(w, d % 32);
      const _Float16 vs = bits2half(((const uint16_t*)A.vscale)[(pg * kPage + t) * NG + g]);
      kh[(r0 + t) * D + d] = half2bits(dq(ck, bits2half(kc[d])));
      vh[(r0 + t) * D + d] = half2bits(dq(cv, vs));
    }
    return;
  }
  const uint16_t* ksrc;
  const uint16_t* vsrc;
  if (A.kivi_packed) {
    const int tp = page - A.n_packed[seq];
    if (tp >= A.tail_pages) return;
    const long tpg = ((long)kvh * A.n_seq + seq) * A.tail_pages + tp;
    ksrc = A.tail_k + tpg * kPage * D;
    vsrc = A.tail_v + tpg * kPage * D;
  } else {
    ksrc = reinterpret_cast<const uint16_t*>(A.kcodes) + pg * kPage * D;
    vsrc = reinterpret_cast<const uint16_t*>(A.vcodes) + pg * kPage * D;
  }
  for (int idx = threadIdx.x; idx < n * D; idx += 64) {
    kh[r0 * D + idx] = ksrc[idx];
    vh[r0 * D + idx] = vsrc[idx];
  }
}

// Row quantizer API (quantizer.py:31-64 + pack_codes_2d).
template <int BITS>
__global__ void quantize_rows_kernel(const uint16_t* __restrict__ x, int rows, int D, int pack, int8_t* codes,
                                     uint16_t* scale) {
  const int G = D / 32;
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * G) return;
  const int r = id / G, g = id % G;
  float v[32];
  int c[32];
  for (int i = 0; i < 32; ++i) v[i] = h2f(x[(long)r * D + g * 32 + i]);
  const _Float16 s = quant_group<BITS>(v, c);
  scale[id] = half2bits(s);
  if (pack) {
    uint32_t w[BITS];
    pack_group<BITS>(c, w);
    int8_t* dst = codes + (long)r * row_bytes(D, BITS) + g * 4 * BITS;
    for (int i = 0; i < 4 * BITS; ++i) dst[i] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
  } else {
    for (int i = 0; i < 32; ++i) codes[(long)r * D + g * 32 + i] = (int8_t)c[i];
  }
}

}  // namespace carekv

// ------------------------------------------------------------------ host side
#include <algorithm>

#include "host_util.h"

using namespace carekv;

// Workspace of carekv_store_pages: per job 4 int32 (counts, then slot
// bases), the call's status word (nonzero when a slot id would fall past the
// arena's n_slots: those slots are dropped, never written), then the store
// pass's staging area (headers, payloads, scales), each part 256-byte aligned.
struct StageLayout {
  int64_t head, kpay, vpay, scale, total;
  int mk, mv;
};
static StageLayout stage_layout(int64_t n_jobs, int D, const carekv_store_params& sp) {
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  StageLayout L;
  store_caps(sp, D / kGroup, &L.mk, &L.mv);
  int64_t o = al(n_jobs * 16 + 16);
  L.head = o;
  o = al(o + n_jobs * 4);
  L.kpay = o;
  o = al(o + n_jobs * L.mk * (kPage * kGroup / 2));
  L.vpay = o;
  o = al(o + n_jobs * L.mv * (kVtb * D / 2));
  L.scale = o;
  o = al(o + n_jobs * (L.mk + L.mv) * 2);
  L.total = o;
  return L;
}
static StoreStage make_stage(void* ws, const StageLayout& L) {
  char* b = static_cast<char*>(ws);
  return StoreStage{reinterpret_cast<uint32_t*>(b + L.head), reinterpret_cast<int8_t*>(b + L.kpay),
                    reinterpret_cast<int8_t*>(b + L.vpay), reinterpret_cast<uint16_t*>(b + L.scale), L.mk, L.mv};
}

extern "C" int64_t carekv_store_workspace_bytes(const carekv_arena* arena, const carekv_store_params* sp,
                                                int32_t n_jobs) {
  if (!arena || !sp || n_jobs < 0) {
    set_error("carekv_store_workspace_bytes: null arena / params or negative n_jobs");
    return -1;
  }
  return stage_layout(n_jobs, arena->head_dim, *sp).total;
}

// Blocks of the store pass: enough to fill the chip several times over;
// each wave then loops over its share of the jobs.
constexpr int kStorePassBlocks = 2048;

template <int D, int BITS, int PATH>
static int launch_pass(const carekv_arena& A, const carekv_store_params& sp, const uint16_t* K, const uint16_t* V,
                       const JobSrc& src, int n_jobs, StoreWs ws, const StoreStage& st, hipStream_t s,
                       const char* what) {
  const int blocks = std::min((n_jobs + 3) / 4, kStorePassBlocks);
  const int lds = store_lds_p_bytes(A.sketch_dim) + 4 * (int)sizeof(StoreLds<D>);
  hipLaunchKernelGGL((store_pages_kernel<D, BITS, PATH>), dim3(blocks), dim3(256), lds, s, A, sp, K, V, src,
                     n_jobs, ws, st);
  CAREKV_CHECK_LAUNCH(what);
  return CAREKV_OK;
}

template <int D>
static int launch_slots(const carekv_arena& A, const JobSrc& src, int n_jobs, int n_groups, StoreWs ws,
                        const StoreStage& st, hipStream_t s) {
  hipLaunchKernelGGL(store_scan_kernel, dim3(n_groups), dim3(1024), 0, s, A, src, ws);
  CAREKV_CHECK_LAUNCH("store_scan");
  hipLaunchKernelGGL((store_slots_kernel<D>), dim3((n_jobs + 15) / 16), dim3(256), 0, s, A, src, n_jobs, ws, st);
  CAREKV_CHECK_LAUNCH("store_slots");
  return CAREKV_OK;
}

// The fp16 tail of a packed KIVI arena as a side-buffer arena under the
// code-page map of n_packed.
static carekv_arena kivi_tail_view(const carekv_arena& A) {
  carekv_arena At = A;
  At.base_bits = 16;
  At.scale_mode = 0;
  At.kcodes = (int8_t*)A.tail_k;
  At.vcodes = (int8_t*)A.tail_v;
  At.kivi_packed = 0;
  At.code_pages = A.tail_pages;
  At.code_page_off = A.n_packed;
  return At;
}

// One call: the store pass (both kinds of page of a packed KIVI arena: the
// packed prefix, then a view of the fp16 tail), the slot scan over all jobs,
// the scatter.
template <int D, int BITS>
static int launch_store(const carekv_arena& A, const carekv_store_params& sp, const uint16_t* K, const uint16_t* V,
                        const JobSrc& src, int n_jobs, int n_groups, StoreWs ws, const StoreStage& st,
                        hipStream_t s) {
  int rc;
  if (A.kivi_packed) {
    rc = launch_pass<D, 2, kPathKivi>(A, sp, K, V, src, n_jobs, ws, st, s, "store_pages (packed KIVI prefix)");
    if (rc == CAREKV_OK)
      rc = launch_pass<D, 16, kPathHat>(kivi_tail_view(A), sp, K, V, src, n_jobs, ws, st, s,
                                        "store_pages (packed KIVI tail)");
  } else if constexpr (BITS == 16) {
    rc = launch_pass<D, 16, kPathHat>(A, sp, K, V, src, n_jobs, ws, st, s, "store_pages (fp16 base)");
  } else if (sp.k_codes_in) {
    rc = launch_pass<D, BITS, kPathCodesIn>(A, sp, K, V, src, n_jobs, ws, st, s, "store_pages (given base)");
  } else if (sp.keep_base) {
    rc = launch_pass<D, BITS, kPathKeep>(A, sp, K, V, src, n_jobs, ws, st, s, "store_pages (kept base)");
  } else {
    rc = launch_pass<D, BITS, kPathFresh>(A, sp, K, V, src, n_jobs, ws, st, s, "store_pages");
  }
  if (rc != CAREKV_OK) return rc;
  return launch_slots<D>(A, src, n_jobs, n_groups, ws, st, s);
}

// Checks and dispatch shared by carekv_store_pages and carekv_store_prefill.
static int store_any(const carekv_arena* arena, const carekv_store_params* sp, const uint16_t* K, const uint16_t* V,
                     const JobSrc& src, int n_jobs, int n_groups, void* workspace, void* stream) {
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.residual_bits == 4, "kernels support residual_bits=4");
  CAREKV_REQUIRE(sp->sketch_proj != nullptr, "sketch_proj is required");
  StoreWs ws{(int32_t*)workspace};
  const StoreStage st = make_stage(workspace, stage_layout(n_jobs, A.head_dim, *sp));
  hipStream_t s = (hipStream_t)stream;
  if (A.kivi_packed) {
    CAREKV_REQUIRE(sp->k_hat && sp->v_hat && sp->k_codes_in && sp->v_codes_in && sp->v_scale_in,
                   "a packed KIVI arena stores from k_hat, v_hat, k_codes_in, v_codes_in and v_scale_in");
    CAREKV_REQUIRE(!sp->keep_base, "keep_base is built for the uniform packed bases");
    if (A.head_dim == 64) return launch_store<64, 2>(A, *sp, K, V, src, n_jobs, n_groups, ws, st, s);
    return launch_store<128, 2>(A, *sp, K, V, src, n_jobs, n_groups, ws, st, s);
  }
  if (A.base_bits == 16) {
    CAREKV_REQUIRE(sp->k_hat && sp->v_hat, "the fp16 base (base_bits=16) needs k_hat and v_hat");
    CAREKV_REQUIRE(!sp->keep_base, "keep_base (streaming store) is built for the packed bases");
    if (A.head_dim == 64) return launch_store<64, 16>(A, *sp, K, V, src, n_jobs, n_groups, ws, st, s);
    return launch_store<128, 16>(A, *sp, K, V, src, n_jobs, n_groups, ws, st, s);
  }
  CAREKV_REQUIRE(!sp->k_codes_in || (sp->k_scale_in && sp->v_codes_in && sp->v_scale_in),
                 "k_codes_in needs k_scale_in, v_codes_in and v_scale_in");
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    return launch_store<decltype(d)::value, decltype(b)::value>(A, *sp, K, V, src, n_jobs, n_groups, ws, st, s);
  });
}

extern "C" int carekv_store_pages(const carekv_arena* arena, const carekv_store_params* sp, const uint16_t* K,
                                  const uint16_t* V, const carekv_page_job* jobs_dev, int32_t n_jobs,
                                  const int32_t* group_ptr_dev, int32_t n_groups, void* workspace,
                                  void* stream) {
  CAREKV_REQUIRE(arena && sp && K && V && jobs_dev && group_ptr_dev && workspace, "null argument");
  CAREKV_REQUIRE(n_jobs >= 0 && n_groups >= 0, "negative sizes");
  if (n_jobs == 0) return CAREKV_OK;
  JobSrc src{};
  src.jobs = jobs_dev;
  src.group_ptr = group_ptr_dev;
  return store_any(arena, sp, K, V, src, n_jobs, n_groups, workspace, stream);
}

extern "C" int carekv_store_prefill(const carekv_arena* arena, const carekv_store_params* sp, const uint16_t* K,
                                    const uint16_t* V, const carekv_prefill_grid* grid, void* workspace,
                                    void* stream) {
  CAREKV_REQUIRE(arena && sp && K && V && grid && grid->rows && workspace, "null argument");
  CAREKV_REQUIRE(grid->n_rows > 0 && grid->n_tokens > 0 && grid->token_start >= 0, "empty or negative grid");
  const int ps = arena->page_size > 0 ? arena->page_size : kPage;
  const int64_t n_pages = (grid->n_tokens + ps - 1) / ps;
  const int64_t n_jobs = (int64_t)grid->n_rows * arena->n_kv_heads * n_pages;
  CAREKV_REQUIRE(n_jobs < (1ll << 31), "grid too large");
  JobSrc src{};
  src.rows = grid->rows;
  src.n_rows = grid->n_rows;
  src.n_kvh = arena->n_kv_heads;
  src.n_pages = (int32_t)n_pages;
  src.n_tokens = grid->n_tokens;
  src.token_start = grid->token_start;
  return store_any(arena, sp, K, V, src, (int)n_jobs, grid->n_rows, workspace, stream);
}

namespace {
int append_any(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* dest_dev,
               int32_t n_rows, const CodedRows& cr, void* stream);
}  // namespace

extern "C" int carekv_append_rows(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows,
                                  const int32_t* dest_dev, int32_t n_rows, void* stream) {
  CAREKV_REQUIRE(k_rows && v_rows, "null argument");
  return append_any(arena, k_rows, v_rows, dest_dev, n_rows, CodedRows{nullptr, nullptr, nullptr, nullptr}, stream);
}

extern "C" int carekv_append_coded_rows(const carekv_arena* arena, const int8_t* k_codes, const uint16_t* k_scale,
                                        const int8_t* v_codes, const uint16_t* v_scale, const int32_t* dest_dev,
                                        int32_t n_rows, void* stream) {
  CAREKV_REQUIRE(k_codes && k_scale && v_codes && v_scale, "null argument");
  CAREKV_REQUIRE(arena && arena->base_bits != 16, "coded rows need a packed base");
  return append_any(arena, nullptr, nullptr, dest_dev, n_rows, CodedRows{k_codes, k_scale, v_codes, v_scale}, stream);
}

namespace {
int append_any(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows, const int32_t* dest_dev,
               int32_t n_rows, const CodedRows& cr, void* stream) {
  CAREKV_REQUIRE(arena && dest_dev, "null argument");
  if (n_rows <= 0) return CAREKV_OK;
  CAREKV_REQUIRE(check_arena(*arena), last_error_buf());
  carekv_arena A = *arena;
  if (A.kivi_packed) {  // decode rows go to the fp16 tail
    CAREKV_REQUIRE(k_rows && v_rows, "a packed KIVI arena appends fp16 rows");
    A = kivi_tail_view(*arena);
  }
  hipStream_t s = (hipStream_t)stream;
  if (A.base_bits == 16) {
    if (A.head_dim == 64)
      hipLaunchKernelGGL(append_hat_rows_kernel<64>, dim3((n_rows + 3) / 4), dim3(256), 0, s, A, k_rows, v_rows,
                         dest_dev, n_rows);
    else
      hipLaunchKernelGGL(append_hat_rows_kernel<128>, dim3((n_rows + 3) / 4), dim3(256), 0, s, A, k_rows, v_rows,
                         dest_dev, n_rows);
    CAREKV_CHECK_LAUNCH("append_hat_rows");
    return CAREKV_OK;
  }
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    hipLaunchKernelGGL((append_rows_kernel<decltype(d)::value, decltype(b)::value>), dim3((n_rows + 3) / 4),
                       dim3(256), 0, s, A, k_rows, v_rows, dest_dev, n_rows, cr);
    CAREKV_CHECK_LAUNCH("append_rows");
    return CAREKV_OK;
  });
}
}  // namespace

extern "C" int carekv_read_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                                 const int32_t* page_ids_dev, const int32_t* row_start_dev, int8_t* kc, uint16_t* ks,
                                 int8_t* vc, uint16_t* vs, void* stream) {
  CAREKV_REQUIRE(arena && row_start_dev && kc && ks && vc && vs, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(seq >= 0 && seq < A.n_seq && kv_head >= 0 && kv_head < A.n_kv_heads, "seq/kv_head out of range");
  CAREKV_REQUIRE(n_pages >= 0 && (page_ids_dev || n_pages <= A.max_pages), "n_pages out of range");
  CAREKV_REQUIRE(A.base_bits != 16 && !A.kivi_packed,
                 "the fp16 and packed KIVI bases have no uniform codes to read: use carekv_read_hat_pages");
  if (n_pages == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_db(A.head_dim, A.base_bits, [&](auto d, auto b) {
    hipLaunchKernelGGL((read_pages_kernel<decltype(d)::value, decltype(b)::value>), dim3(n_pages), dim3(64), 0, s,
                       A, seq, kv_head, n_pages, page_ids_dev, row_start_dev, kc, ks, vc, vs);
    CAREKV_CHECK_LAUNCH("read_pages");
    return CAREKV_OK;
  });
}

extern "C" int carekv_quantize_rows(const uint16_t* x, int32_t rows, int32_t D, int32_t bits, int32_t group,
                                    int32_t pack, int8_t* codes, uint16_t* scale, void* stream) {
  CAREKV_REQUIRE(x && codes && scale, "null argument");
  CAREKV_REQUIRE(group == 32 && D % 32 == 0 && D > 0, "kernels support group_size=32 and D % 32 == 0");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  if (rows <= 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const int n = rows * (D / 32);
  const int blocks = (n + 255) / 256;
  switch (bits) {
    case 2: hipLaunchKernelGGL(quantize_rows_kernel<2>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
    case 3: hipLaunchKernelGGL(quantize_rows_kernel<3>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
    default: hipLaunchKernelGGL(quantize_rows_kernel<4>, dim3(blocks), dim3(256), 0, s, x, rows, D, pack, codes, scale); break;
  }
  CAREKV_CHECK_LAUNCH("quantize_rows");
  return CAREKV_OK;
}

extern "C" int carekv_kivi_codes(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits,
                                 int32_t per_channel, int8_t* codes, uint16_t* scale, void* stream) {
  CAREKV_REQUIRE(x && codes && scale, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D <= 1024 && n_mat >= 0 && rows >= 0, "bad shape");
  if (n_mat == 0 || rows == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (per_channel) {
    CAREKV_REQUIRE(n_mat <= 65535 * 1024, "too many matrices");
    hipLaunchKernelGGL(kivi_channel_codes_kernel, dim3(n_mat, (D + 63) / 64), dim3(256), 0, s, x, rows, D, bits,
                       codes, scale);
  } else {
    const long n_rows = (long)n_mat * rows;
    CAREKV_REQUIRE((n_rows + 3) / 4 <= 0x7fffffffL, "too many rows");
    hipLaunchKernelGGL(kivi_token_codes_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, s, x, n_rows, D,
                       bits, codes, scale);
  }
  CAREKV_CHECK_LAUNCH("kivi_codes");
  return CAREKV_OK;
}

extern "C" int carekv_read_hat_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                                     const int32_t* page_ids_dev, const int32_t* row_start_dev, uint16_t* k_hat,
                                     uint16_t* v_hat, void* stream) {
  CAREKV_REQUIRE(arena && row_start_dev && k_hat && v_hat, "null argument");
  const carekv_arena& A = *arena;
  CAREKV_REQUIRE(check_arena(A), last_error_buf());
  CAREKV_REQUIRE(A.base_bits == 16 || A.kivi_packed, "carekv_read_hat_pages reads the fp16 and packed KIVI bases");
  CAREKV_REQUIRE(seq >= 0 && seq < A.n_seq && kv_head >= 0 && kv_head < A.n_kv_heads, "seq/kv_head out of range");
  CAREKV_REQUIRE(n_pages >= 0 && (page_ids_dev || n_pages <= A.max_pages), "n_pages out of range");
  if (n_pages == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (A.head_dim == 64)
    hipLaunchKernelGGL(read_hat_pages_kernel<64>, dim3(n_pages), dim3(64), 0, s, A, seq, kv_head, n_pages,
                       page_ids_dev, row_start_dev, k_hat, v_hat);
  else
    hipLaunchKernelGGL(read_hat_pages_kernel<128>, dim3(n_pages), dim3(64), 0, s, A, seq, kv_head, n_pages,
                       page_ids_dev, row_start_dev, k_hat, v_hat);
  CAREKV_CHECK_LAUNCH("read_hat_pages");
  return CAREKV_OK;
}

extern "C" int carekv_kivi_qdq(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits,
                               int32_t per_channel, uint16_t* out, void* stream) {
  CAREKV_REQUIRE(x && out, "null argument");
  CAREKV_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3 or 4");
  CAREKV_REQUIRE(D > 0 && D <= 1024 && n_mat >= 0 && rows >= 0, "bad shape");
  if (n_mat == 0 || rows == 0) return CAREKV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (per_channel) {
    CAREKV_REQUIRE(n_mat <= 65535 * 1024, "too many matrices");
    hipLaunchKernelGGL(kivi_channel_kernel, dim3(n_mat, (D + 63) / 64), dim3(256), 0, s, x, rows, D, bits, out);
  } else {
    const long n_rows = (long)n_mat * rows;
    CAREKV_REQUIRE((n_rows + 3) / 4 <= 0x7fffffffL, "too many rows");
    hipLaunchKernelGGL(kivi_token_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, s, x, n_rows, D, bits, out);
  }
  CAREKV_CHECK_LAUNCH("kivi_qdq");
  return CAREKV_OK;
}
