// Per-page building blocks shared by the streaming and apply kernels of the
// decode (gfx950, wave64).  A wave works on one 16-token page at a time;
// lane l = 16*j + m holds token m, dims [j*D/4, (j+1)*D/4) of the page when
// it loads codes, and query column m, tokens 4j..4j+3 in MFMA results.
#pragma once

#include "decode_common.h"

namespace carekv {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(4))) int32_t cint32_t;  // read-only, scalar loads when uniform

constexpr uint32_t kBufFlags = 0x00020000u;  // raw buffer resource word 3 (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kBufFlags);
}

__device__ __forceinline__ float4_t mfma16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// x[l] op x[l ^ 16] and x[l] op x[l ^ 32] through the gfx950 lane-swap
// instructions: both results hold the pair {x[l], x[l^16]} (resp. ^32) in
// some order, and the ops used are commutative, so the lanes of a pair end
// with identical bits.
__device__ __forceinline__ float pair16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Reduce three per-lane values over the 4 lane groups j = l / 16 with three
// lane swaps: afterwards group 0 holds sum(a), group 1 sum(b), groups 2
// and 3 sum(c).  permlane16_swap(X, Y) exchanges the odd 16-lane rows of X
// with the even rows of Y; permlane32_swap(X, Y) the upper half of X with
// the lower half of Y.
__device__ __forceinline__ float moments_reduce(float a, float b, float c) {
  const auto ab = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float x = __uint_as_float(ab[0]) + __uint_as_float(ab[1]);  // even rows: a pair sum, odd rows: b
  const float cc = pair16_sum(c);
  const auto xc = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(cc), false, false);
  return __uint_as_float(xc[0]) + __uint_as_float(xc[1]);  // lower half: x total, upper half: c total
}

// Four values reduced the same way: group j ends with the sum of the j-th.
__device__ __forceinline__ float moments_reduce4(float a, float b, float c, float d) {
  const auto ab = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float x = __uint_as_float(ab[0]) + __uint_as_float(ab[1]);  // even rows: a pair sum, odd rows: b
  const auto cd = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  const float y = __uint_as_float(cd[0]) + __uint_as_float(cd[1]);  // even rows: c pair sum, odd rows: d
  const auto xy = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(xy[0]) + __uint_as_float(xy[1]);  // rows 0..3: a, b, c, d totals
}

// Sum over the four lanes m, m+16, m+32, m+48 (the token groups of a query).
__device__ __forceinline__ float col_sum(float v) { return pair32_sum(pair16_sum(v)); }
__device__ __forceinline__ float col_max(float v) { return pair32_max(pair16_max(v)); }

// ---------------------------------------------------------------- code pairs
// A chunk of NC codes (FB-bit two's complement fields of a little-endian
// bit string) is decoded two codes at a time into fp16 pairs.  The pairs are
// (blk + k, blk + k + PD) inside blocks of BLK codes (geometry of schedule
// SB); the pair order fixes the order of the reduction dimension of the
// MFMAs that consume them.  A pair is masked out of 32-bit windows of the
// bit string into the mantissas of two fp16 values 1024 + u * 2^o
// (u = offset-binary code, o = field offset), after which one packed FMA
// gives the two signed codes exactly.
template <int SB> struct PairGeom;
template <> struct PairGeom<2> { static constexpr int BLK = 16, PD = 8; };
template <> struct PairGeom<3> { static constexpr int BLK = 8, PD = 4; };
template <> struct PairGeom<4> { static constexpr int BLK = 8, PD = 4; };
template <> struct PairGeom<16> { static constexpr int BLK = 2, PD = 1; };  // natural order (fp16 base)

template <int FB, int NC, int SB>
struct Pairs {
  static constexpr int NP = NC / 2;
  static constexpr int NW = (NC * FB + 31) / 32;
  static constexpr int MAXO = 10 - FB;  // field must stay inside the 10-bit mantissa
  struct Tab {
    int a[NP], b[NP];      // code indices of the pair
    int Wa[NP], Wb[NP];    // window start bits of the low / high field
    int ha[NP], hb[NP];    // highest bit any user of that window needs
    int ao[NP], bo[NP];    // field offsets inside the low / high halves
    int slot_code[NC];     // fp16 slot 2i (+1) -> code a_i (b_i)
  };
  static constexpr Tab make() {
    Tab t{};
    constexpr int BLK = PairGeom<SB>::BLK, PD = PairGeom<SB>::PD;
    constexpr int NONE = -100000;
    int n = 0, W = NONE, WA = NONE, WB = NONE;
    for (int blk = 0; blk < NC; blk += BLK)
      for (int k = 0; k < BLK / 2; ++k) {
        const int ia = blk + k, ib = ia + PD;
        const int ba = FB * ia, bb = FB * ib;
        t.a[n] = ia; t.b[n] = ib;
        t.slot_code[2 * n] = ia; t.slot_code[2 * n + 1] = ib;
        const int lo_a = ba - MAXO, hi_a = ba;            // Wa range: ao in [0, MAXO]
        const int lo_b = bb - 16 - MAXO, hi_b = bb - 16;  // Wb range: bo in [0, MAXO]
        const int lo = lo_a > lo_b ? lo_a : lo_b, hi = hi_a < hi_b ? hi_a : hi_b;
        if (lo <= hi) {  // one window serves both fields
          if (!(W >= lo && W <= hi)) W = hi;
          t.Wa[n] = t.Wb[n] = W;
        } else {  // two windows
          W = NONE;
          if (!(WA >= lo_a && WA <= hi_a)) WA = hi_a;
          if (!(WB >= lo_b && WB <= hi_b)) WB = hi_b;
          t.Wa[n] = WA; t.Wb[n] = WB;
        }
        t.ao[n] = ba - t.Wa[n];
        t.bo[n] = bb - 16 - t.Wb[n];
        ++n;
      }
    // highest needed bit per distinct window value
    for (int i = 0; i < NP; ++i) {
      int h_a = 0, h_b = 0;
      for (int j = 0; j < NP; ++j) {
        const int na = FB * t.a[j] + FB - 1, nb = FB * t.b[j] + FB - 1;
        if (t.Wa[j] == t.Wa[i] && na > h_a) h_a = na;
        if (t.Wb[j] == t.Wa[i] && nb > h_a) h_a = nb;
        if (t.Wa[j] == t.Wb[i] && na > h_b) h_b = na;
        if (t.Wb[j] == t.Wb[i] && nb > h_b) h_b = nb;
      }
      t.ha[i] = h_a; t.hb[i] = h_b;
    }
    return t;
  }
  static constexpr Tab T = make();
};

// The fp16 side-buffer base (BITS = 16, base_quantizer kivi_style): the
// "codes" are the K_hat / V_hat values themselves, pair i = 32-bit word i.
template <int NC>
struct Pairs<16, NC, 16> {
  static constexpr int NP = NC / 2;
  struct Tab {
    int a[NP], b[NP];  // code indices of pair i: 2i, 2i + 1
    int slot_code[NC];
  };
  static constexpr Tab make() {
    Tab t{};
    for (int i = 0; i < NP; ++i) { t.a[i] = 2 * i; t.b[i] = 2 * i + 1; }
    for (int i = 0; i < NC; ++i) t.slot_code[i] = i;
    return t;
  }
  static constexpr Tab T = make();
};

// 32-bit window of the bit string in w starting at bit W (may be negative);
// bits above `hi` are not needed.
template <int NW>
__device__ __forceinline__ uint32_t window(const uint32_t* w, int W, int hi) {
  if (W < 0) return w[0] << (-W);
  const int d = W >> 5, s = W & 31;
  if (s == 0) return w[d];
  if (hi < 32 * (d + 1) || d + 1 >= NW) return w[d] >> s;
  return __builtin_amdgcn_alignbit(w[d + 1], w[d], s);
}

// Pair i of the chunk as two exact signed codes in fp16.
template <int FB, int NC, int SB>
__device__ __forceinline__ half2_t code_pair(const uint32_t* w, int i) {
  using P = Pairs<FB, NC, SB>;
  constexpr uint32_t fm = (1u << FB) - 1u, top = 1u << (FB - 1);
  const int ao = P::T.ao[i], bo = P::T.bo[i];
  const uint32_t ma = fm << ao, mb = fm << (16 + bo);
  const uint32_t fa = top << ao, fb = top << (16 + bo);  // two's complement -> offset binary
  uint32_t x;
  if (P::T.Wa[i] == P::T.Wb[i]) {
    const uint32_t v = window<P::NW>(w, P::T.Wa[i], P::T.ha[i]);
    x = ((v ^ (fa | fb)) & (ma | mb)) | 0x64006400u;
  } else {
    const uint32_t va = window<P::NW>(w, P::T.Wa[i], P::T.ha[i]);
    const uint32_t vb = window<P::NW>(w, P::T.Wb[i], P::T.hb[i]);
    x = ((va ^ fa) & ma) | ((vb ^ fb) & mb) | 0x64006400u;
  }
  half2_t v;
  __builtin_memcpy(&v, &x, 4);
  const half2_t sc = {(_Float16)(1.0f / (float)(1 << ao)), (_Float16)(1.0f / (float)(1 << bo))};
  const half2_t of = {(_Float16)(-(1024.0f / (float)(1 << ao) + (float)top)),
                      (_Float16)(-(1024.0f / (float)(1 << bo) + (float)top))};
  return __builtin_elementwise_fma(v, sc, of);
}

// Pair i of the chunk as two offset-binary codes u = code + 2^(FB-1) held as
// fp16 subnormals u * 2^(o - 24), o = the field's offset inside its half
// (the masked field without exponent bits): one bitop3 per window.  MFMA
// products of these with fp16 weights are exact in fp32; the consumer
// scales slot s by 2^(24 - o(s)) (slot_off) and subtracts 2^(FB-1) times
// the sum of the weights it applied.
template <int FB, int NC, int SB>
__device__ __forceinline__ uint32_t code_pair_sub(const uint32_t* w, int i) {
  using P = Pairs<FB, NC, SB>;
  constexpr uint32_t fm = (1u << FB) - 1u, top = 1u << (FB - 1);
  const int ao = P::T.ao[i], bo = P::T.bo[i];
  const uint32_t ma = fm << ao, mb = fm << (16 + bo);
  const uint32_t fa = top << ao, fb = top << (16 + bo);
  if (P::T.Wa[i] == P::T.Wb[i]) {
    const uint32_t v = window<P::NW>(w, P::T.Wa[i], P::T.ha[i]);
    return (v ^ (fa | fb)) & (ma | mb);
  }
  const uint32_t va = window<P::NW>(w, P::T.Wa[i], P::T.ha[i]);
  const uint32_t vb = window<P::NW>(w, P::T.Wb[i], P::T.hb[i]);
  return ((va ^ fa) & ma) | ((vb ^ fb) & mb);
}

// Exact half(code * s) for all pairs of the chunk (quantizer.py:67-82: the
// product code*s is exact in fp32 and rounded once to fp16; the packed fp16
// multiply of the exact code rounds the same exact product once).
template <int FB, int NC, int SB>
__device__ __forceinline__ void dequant_pairs(const uint32_t* w, _Float16 s, half2_t* out) {
  if constexpr (FB == 16) {  // fp16 base: the values themselves, no scale
#pragma unroll
    for (int i = 0; i < NC / 2; ++i) __builtin_memcpy(&out[i], &w[i], 4);
  } else {
    const half2_t ss = {s, s};
#pragma unroll
    for (int i = 0; i < NC / 2; ++i) out[i] = code_pair<FB, NC, SB>(w, i) * ss;
  }
}

__device__ __forceinline__ uint32_t h2bits(half2_t v) {
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

// Buffer load of N bytes (N = 4, 6, 8, 12, 16 or a multiple of 16) at byte offset off.
template <int N>
__device__ __forceinline__ void buf_load(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (N > 16 && N % 16 == 0) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      w[4 * i] = v[0]; w[4 * i + 1] = v[1]; w[4 * i + 2] = v[2]; w[4 * i + 3] = v[3];
    }
  } else if constexpr (N == 16) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (N == 12) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2];
  } else if constexpr (N == 8) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    w[0] = v[0]; w[1] = v[1];
  } else if constexpr (N == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else {
    static_assert(N == 6, "chunk size");
    const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    const uint32_t mid = __builtin_amdgcn_raw_buffer_load_b16(r, off + 2, 0, 0);
    const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(r, off + 4, 0, 0);
    w[0] = lo | (mid << 16);
    w[1] = hi;
  }
}

// ---------------------------------------------------------------- geometry
template <int D, int BITS>
struct PageGeom {
  static constexpr int CH = D / 4;              // codes per lane (quarter row)
  static constexpr int CHB = CH * BITS / 8;     // packed bytes per lane
  static constexpr int NWC = (CHB + 3) / 4;     // 32-bit words per lane chunk
  static constexpr int RB = row_bytes(D, BITS); // packed bytes per row
  static constexpr int NCG = D / 32;            // K channel groups / scale groups
  static constexpr int NS = CH / 8;             // 16x16x32 MFMA steps for S
  static constexpr int NT = D / 16;             // PV output tiles
  static constexpr int VROW = D / 2 + 4;        // V tile row stride in words (padded)
  static constexpr int KSB = kPage * 32 / 2;    // K residual slot bytes
  static constexpr int VSB = kVtb * D / 2;      // V residual slot bytes
  using PB = Pairs<BITS, CH, BITS>;             // base codes
  using PR = Pairs<4, CH, BITS>;                // V residual codes, base pair order
  using PK = Pairs<4, 8, 4>;                    // K residual codes (8 per lane)
};

// Row resources of one (kv head, sequence): codes and scales of its pages.
struct RowRes {
  __amdgpu_buffer_rsrc_t kc, vc, ks, vs;
};

// pg_end clamps the resources at that page of the row: a load past it
// returns 0 without a memory access.  On a view with a code-page map
// (carekv_arena::code_pages; fp16 pages only) the resources start at the
// row's code pages shifted back by its offset, so page p still loads at
// p * page bytes; the caller touches only pages the map holds.
template <int D, int BITS, int SM>
__device__ __forceinline__ RowRes row_resources(const carekv_arena& A, long pg_base, int pg_end = -1) {
  using G = PageGeom<D, BITS>;
  long cb = pg_base;
  int lim = A.max_pages;
  if constexpr (BITS == 16) {  // maps hold fp16 pages only (the tail of a packed KIVI arena)
    if (A.code_pages > 0) {
      cb = code_base(A, pg_base);
      lim = code_page_limit(A, pg_base);
    }
  }
  const uint32_t rows = (uint32_t)(pg_end >= 0 ? min(pg_end, lim) : lim) * kPage;
  constexpr int ssz = SM == 1 ? 1 : 2;
  RowRes r;
  r.kc = make_rsrc(A.kcodes + cb * kPage * G::RB, rows * G::RB);
  r.vc = make_rsrc(A.vcodes + cb * kPage * G::RB, rows * G::RB);
  if constexpr (BITS == 16) {  // no scales: empty resources, loads return 0
    r.ks = make_rsrc(nullptr, 0u);
    r.vs = make_rsrc(nullptr, 0u);
  } else {
    r.ks = make_rsrc((const char*)A.kscale + cb * kPage * G::NCG * ssz, rows * G::NCG * ssz);
    r.vs = make_rsrc((const char*)A.vscale + cb * kPage * G::NCG * ssz, rows * G::NCG * ssz);
  }
  return r;
}

// Lane's share of one page: packed codes and raw scale codes of its token
// and quarter row.
template <int D, int BITS>
struct PageRegs {
  uint32_t kw[PageGeom<D, BITS>::NWC], vw[PageGeom<D, BITS>::NWC];
  int ksc, vsc;
};

template <int D, int BITS, int SM>
__device__ __forceinline__ void load_page_regs(PageRegs<D, BITS>& r, const RowRes& rr, int p, int ln, int lj) {
  using G = PageGeom<D, BITS>;
  const uint32_t row = (uint32_t)(p * kPage + ln);
  buf_load<G::CHB>(r.kw, rr.kc, row * G::RB + lj * G::CHB);
  buf_load<G::CHB>(r.vw, rr.vc, row * G::RB + lj * G::CHB);
  const int gi = (lj * G::CH) / 32;
  if constexpr (SM == 1) {
    r.ksc = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rr.ks, row * G::NCG + gi, 0, 0);
    r.vsc = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rr.vs, row * G::NCG + gi, 0, 0);
  } else {
    r.ksc = __builtin_amdgcn_raw_buffer_load_b16(rr.ks, (row * G::NCG + gi) * 2, 0, 0);
    r.vsc = __builtin_amdgcn_raw_buffer_load_b16(rr.vs, (row * G::NCG + gi) * 2, 0, 0);
  }
}

// Scale of the lane's (token, group): int8 code read back as
// half(code * master) (cache.py:713-718, SM = 1) or the raw fp16 scale.
template <int SM>
__device__ __forceinline__ _Float16 lane_scale(int code, float master) {
  if constexpr (SM == 1) return (_Float16)((float)code * master);
  else return bits2half((uint16_t)code);
}

// Uniform per-page metadata (scalar registers).
template <int NCG>
struct PageMeta {
  int nv, meta;
  int ksl[NCG], vsl[kVtb];
  uint32_t kmaster, vmaster;  // fp16 bits (int8 scale mode)
};

// The metadata of a page spread over the lanes of one VGPR (lane 0 valid,
// 1 has_meta, 2.. k_slot, 6..9 v_slot, 10/11 the fp16 masters): vector
// loads, so a prefetch of the next page stays in flight while the wave
// waits for its own LDS traffic (scalar loads share the LDS wait counter).
template <int NCG>
__device__ __forceinline__ int meta_lanes_load(const carekv_arena& A, long pg, int lane) {
  int v = 0;
  if (lane == 0) v = A.valid[pg];
  else if (lane == 1) v = A.has_meta[pg];
  else if (lane < 2 + NCG) v = A.k_slot[pg * NCG + lane - 2];
  else if (lane >= 6 && lane < 10) v = A.v_slot[pg * kVtb + lane - 6];
  else if (lane == 10 && A.scale_mode == 1) v = A.kmaster[pg];
  else if (lane == 11 && A.scale_mode == 1) v = A.vmaster[pg];
  return v;
}

// Slot ids outside the arena read as "no slot".
template <int NCG>
__device__ __forceinline__ PageMeta<NCG> meta_from_lanes(int v, const carekv_arena& A) {
  PageMeta<NCG> m;
  m.nv = __builtin_amdgcn_readlane(v, 0);
  m.meta = __builtin_amdgcn_readlane(v, 1);
#pragma unroll
  for (int c = 0; c < NCG; ++c) {
    const int s = __builtin_amdgcn_readlane(v, 2 + c);
    m.ksl[c] = s < A.n_slots ? s : -1;
  }
#pragma unroll
  for (int b = 0; b < kVtb; ++b) {
    const int s = __builtin_amdgcn_readlane(v, 6 + b);
    m.vsl[b] = s < A.n_slots ? s : -1;
  }
  m.kmaster = (uint32_t)__builtin_amdgcn_readlane(v, 10) & 0xffffu;
  m.vmaster = (uint32_t)__builtin_amdgcn_readlane(v, 11) & 0xffffu;
  return m;
}

// S[token 4j+i][query m] += K_hat . q for the page (NS MFMA 16x16x32 steps).
template <int D, int BITS>
__device__ __forceinline__ float4_t page_scores(const uint32_t* kw, _Float16 ks, const half8_t* qB) {
  using G = PageGeom<D, BITS>;
  half2_t kp[G::CH / 2];
  dequant_pairs<BITS, G::CH, BITS>(kw, ks, kp);
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < G::NS; ++s) {
    const half8_t ak = {kp[4 * s][0], kp[4 * s][1], kp[4 * s + 1][0], kp[4 * s + 1][1],
                        kp[4 * s + 2][0], kp[4 * s + 2][1], kp[4 * s + 3][0], kp[4 * s + 3][1]};
    acc = mfma16x32(ak, qB[s], acc);
  }
  return acc;
}

// q in the order of the page_scores reduction: lane (m = query, j) holds
// q_m at the dims of step s of its chunk.
template <int D, int BITS>
__device__ __forceinline__ void load_q_operand(half8_t* qB, const _Float16* sq, int ln, int lj) {
  using G = PageGeom<D, BITS>;
  using P = typename G::PB;
  const _Float16* qp = sq + ln * D + lj * G::CH;
#pragma unroll
  for (int s = 0; s < G::NS; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) qB[s][e] = qp[P::T.slot_code[8 * s + e]];
}

// V tile rows in LDS: row m = token, CH/2 fp16 pairs per lane chunk, in
// the slot order of the base pair schedule.
template <int D, int BITS>
__device__ __forceinline__ void vtile_write(uint32_t* vt, const half2_t* vp, int ln, int lj) {
  using G = PageGeom<D, BITS>;
  uint32_t* dst = vt + ln * G::VROW + lj * (G::CH / 2);
#pragma unroll
  for (int i = 0; i < G::CH / 2; i += 4)
    *reinterpret_cast<uint4*>(dst + i) = make_uint4(h2bits(vp[i]), h2bits(vp[i + 1]), h2bits(vp[i + 2]),
                                                    h2bits(vp[i + 3]));
}

template <int D, int BITS>
__device__ __forceinline__ void vtile_write_raw(uint32_t* vt, const uint32_t* vp, int ln, int lj) {
  using G = PageGeom<D, BITS>;
  uint32_t* dst = vt + ln * G::VROW + lj * (G::CH / 2);
#pragma unroll
  for (int i = 0; i < G::CH / 2; i += 4) *reinterpret_cast<uint4*>(dst + i) = make_uint4(vp[i], vp[i + 1], vp[i + 2], vp[i + 3]);
}

// acc[t] += P V_tile on MFMA 16x16x16: tile t, column n stands for slot
// 16t + n; k = the page's 16 tokens, P in the A layout (lane (m, j) holds
// P[query m][token 4j+i]).  The B operand (tokens 4j..4j+3 of one slot
// column per lane) comes straight from the token-major tile through the
// gfx950 transpose load: in each 16-lane group, output lane i receives
// element i % 4 of the 4-half rows read by lanes i/4, i/4+4, i/4+8,
// i/4+12, so lane r of group j reads row 4j + r/4, slots 4(r%4) .. +3 of
// the tile's 16.
template <int D, int BITS>
__device__ __forceinline__ void pv_accumulate(const uint32_t* vt, half4_t ap, float4_t* acc, int ln, int lj) {
  using G = PageGeom<D, BITS>;
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  const __attribute__((address_space(3))) char* base =
      (const __attribute__((address_space(3))) char*)vt + ((4 * lj + (ln >> 2)) * G::VROW) * 4 + (ln & 3) * 8;
#pragma unroll
  for (int t = 0; t < G::NT; ++t) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + 32 * t));
    half4_t bv;
    __builtin_memcpy(&bv, &v, 8);
    acc[t] = mfma16(ap, bv, acc[t]);
  }
}

// pv_accumulate with weights carried as hi + lo fp16 pairs (w = hi + lo to
// about 22 bits): the tile is read once and met by both halves.  Used where
// fp16 weights lose too much, e.g. correction weights a_t (e^dS - 1) that
// multiply wide V rows and partly cancel against O_base.
template <int D, int BITS>
__device__ __forceinline__ void pv_accumulate2(const uint32_t* vt, half4_t ah, half4_t al, float4_t* acc, int ln,
                                               int lj) {
  using G = PageGeom<D, BITS>;
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  const __attribute__((address_space(3))) char* base =
      (const __attribute__((address_space(3))) char*)vt + ((4 * lj + (ln >> 2)) * G::VROW) * 4 + (ln & 3) * 8;
#pragma unroll
  for (int t = 0; t < G::NT; ++t) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + 32 * t));
    half4_t bv;
    __builtin_memcpy(&bv, &v, 8);
    acc[t] = mfma16(al, bv, acc[t]);
    acc[t] = mfma16(ah, bv, acc[t]);
  }
}

// Split fp32 weights into fp16 hi + lo (lo = the rounding error of hi).
__device__ __forceinline__ void split_weights(const float (&c)[4], half4_t& hi, half4_t& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = (_Float16)c[i];
    lo[i] = (_Float16)(c[i] - (float)hi[i]);
  }
}

// dS numerator of one K residual slot: racc[i] = sum_d code[token 4j+i][d] *
// q_m[cg*32 + d] (exact codes, fp32 accumulation); the caller applies the
// slot scale.  The slot holds 16 rows of 32 4-bit codes (16 bytes a row);
// word = bytes 4j..4j+3 of row m (codes 8j..8j+7).  sqr holds q in the
// residual pair order (stage_q).
__device__ __forceinline__ float4_t kslot_dot_w(uint32_t word, const _Float16* sqr, int D, int cg, int ln, int lj) {
  const uint32_t w[1] = {word};
  half8_t ar;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half2_t c = code_pair<4, 8, 4>(w, i);
    ar[2 * i] = c[0];
    ar[2 * i + 1] = c[1];
  }
  const half8_t bq = *reinterpret_cast<const half8_t*>(sqr + ln * D + cg * 32 + 8 * lj);
  const float4_t z = {0.f, 0.f, 0.f, 0.f};
  return mfma16x32(ar, bq, z);
}

__device__ __forceinline__ float4_t kslot_dot(const int8_t* slot_base, const _Float16* sqr, int D, int cg, int ln,
                                              int lj) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(slot_base, kPage * 16);
  return kslot_dot_w(__builtin_amdgcn_raw_buffer_load_b32(r, ln * 16 + lj * 4, 0, 0), sqr, D, cg, ln, lj);
}

// Stage the GQ query rows of (b, kv head) in LDS as fp16 [16][D] (rows >= GQ
// zero), in natural order (sq) and in the pair order of the K residual
// codes inside every 8-dim block (sqr).  Call with all threads of the
// block, followed by a barrier.
// rowp(n) gives query row n (nullptr: a zero row).
template <int D, class RowPtr>
__device__ __forceinline__ void stage_q_by(_Float16* sq, _Float16* sqr, RowPtr rowp) {
  using P = Pairs<4, 8, 4>;
  for (int i = threadIdx.x; i < 16 * D; i += blockDim.x) {
    const int n = i / D, d = i % D;
    const uint16_t* r = rowp(n);
    sq[i] = r ? bits2half(r[d]) : (_Float16)0.f;
    sqr[i] = r ? bits2half(r[(d & ~7) + P::T.slot_code[d & 7]]) : (_Float16)0.f;
  }
}
template <int D>
__device__ __forceinline__ void stage_q(_Float16* sq, _Float16* sqr, const uint16_t* q, int GQ) {
  stage_q_by<D>(sq, sqr, [&](int n) { return n < GQ ? q + n * D : (const uint16_t*)nullptr; });
}

// Merge the 4 waves' online-softmax partials (m, l, O rows = queries) into
// one split partial: po[q][d] = sum_w O_w[q][d] 2^(m_w - M), pml[q] = (M, L).
// O comes in the PV accumulator layout (tile t, lane (n, j): rows 4j+i,
// column n = slot 16t + n).  Two rounds of D/2 dims through so[4][16][D/2].
// Call with all threads of the block.
template <int D, int BITS>
__device__ __forceinline__ void merge_waves(float* so, float (*s_m)[16], float (*s_l)[16], float m_run,
                                            float l_run, const float4_t* oacc, int w, int ln, int lj, int GQ,
                                            float* po, float* pml) {
  using G = PageGeom<D, BITS>;
  constexpr int NT = G::NT, CH = G::CH, DH = D / 2;
  __syncthreads();
  if (lj == 0) { s_m[w][ln] = m_run; s_l[w][ln] = l_run; }
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int slot = 16 * t + ln;
      const int dim = (slot / CH) * CH + G::PB::T.slot_code[slot % CH];
      if ((dim >= DH) != (half == 1)) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) so[(w * 16 + 4 * lj + i) * DH + dim - half * DH] = oacc[t][i];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < GQ * DH; idx += blockDim.x) {
      const int qq = idx / DH, d = idx % DH;
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][qq]);
      float L = 0.f, O = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
          const float f = __builtin_amdgcn_exp2f(s_m[ww][qq] - M);
          L += s_l[ww][qq] * f;
          O += so[(ww * 16 + qq) * DH + d] * f;
        }
      }
      po[qq * D + half * DH + d] = O;
      if (half == 0 && d == 0) { pml[qq * 2] = M; pml[qq * 2 + 1] = L; }
    }
    __syncthreads();
  }
}

// Sum the 4 waves' PV accumulators (rows = queries) into out[q][d] (fixed
// wave order), two rounds of D/2 dims through so[4][16][D/2].  Call with all
// threads of the block.
template <int D, int BITS>
__device__ __forceinline__ void sum_waves(float* so, const float4_t* acc, int w, int ln, int lj, int GQ, float* out) {
  using G = PageGeom<D, BITS>;
  constexpr int NT = G::NT, CH = G::CH, DH = D / 2;
  __syncthreads();
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int slot = 16 * t + ln;
      const int dim = (slot / CH) * CH + G::PB::T.slot_code[slot % CH];
      if ((dim >= DH) != (half == 1)) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) so[(w * 16 + 4 * lj + i) * DH + dim - half * DH] = acc[t][i];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < GQ * DH; idx += blockDim.x) {
      const int qq = idx / DH, d = idx % DH;
      out[qq * D + half * DH + d] = ((so[qq * DH + d] + so[(16 + qq) * DH + d]) + so[(32 + qq) * DH + d]) +
                                    so[(48 + qq) * DH + d];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- 4x4x4 layout helpers
__device__ __forceinline__ float4_t mfma4x4(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

// v from lane (i + N) % 16 of the same 16-lane row (DPP row rotate)
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}
// Sum / max over the lanes {i, i+4, i+8, i+12} of each 16-lane row.
__device__ __forceinline__ float row4_sum(float v) {
  v += row_ror<4>(v);
  return v + row_ror<8>(v);
}
__device__ __forceinline__ float row4_max(float v) {
  v = fmaxf(v, row_ror<4>(v));
  return fmaxf(v, row_ror<8>(v));
}

// Max / min reductions on integers: one DPP or lane-swap op per step, where
// the float max needs its inputs canonicalised first.
template <int N>
__device__ __forceinline__ int row_ror_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xf, 0xf, false);
}
__device__ __forceinline__ int row4_max_i(int v) {
  v = max(v, row_ror_i<4>(v));
  return max(v, row_ror_i<8>(v));
}
__device__ __forceinline__ int row4_min_i(int v) {
  v = min(v, row_ror_i<4>(v));
  return min(v, row_ror_i<8>(v));
}
__device__ __forceinline__ int pair16_max_i(int v) {
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  return max((int)r[0], (int)r[1]);
}
__device__ __forceinline__ int pair32_max_i(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return max((int)r[0], (int)r[1]);
}
// Order key of a float: the signed-integer order of the keys is the float
// order for every value but NaN (-0 sorts just below +0); its own inverse.
__device__ __forceinline__ int fkey(float f) {
  const int b = __float_as_int(f);
  return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float fkey_inv(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7fffffff)); }

__device__ __forceinline__ uint32_t pack_h2(float x, float y) {
  const half2_t h = {(_Float16)x, (_Float16)y};
  return h2bits(h);
}

// Buffer load of a packed row of N bytes (N a multiple of 8) at byte offset off.
template <int N>
__device__ __forceinline__ void buf_load_row(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (N % 16 == 0) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      w[4 * i] = v[0]; w[4 * i + 1] = v[1]; w[4 * i + 2] = v[2]; w[4 * i + 3] = v[3];
    }
  } else {
    static_assert(N % 8 == 0, "row bytes");
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off + 8 * i, 0, 0);
      w[2 * i] = v[0]; w[2 * i + 1] = v[1];
    }
  }
}

// *(T*)(base + off) with a 32-bit byte offset (base uniform).
template <typename T>
__device__ __forceinline__ T ld_off(const void* base, uint32_t off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + off);
}

// Field f of page p of a row (the lane layout of meta_lanes_load: 0 valid,
// 1 has_meta, 2.. the K slots, 6..9 the V slots, 10 / 11 the K / V scale
// masters), 0 when the page is not ok.  Every load is on a row base
// (uniform) plus a 32-bit lane index: five loads per lane (valid, k_slot,
// v_slot, master, has_meta) and a select of values, so no per-lane 64-bit
// address stays live; a lane whose field is in another array, or whose page
// is not ok, reads page 0 of the row (always mapped) and drops the value.
template <int NCG, int SM>
__device__ __forceinline__ int meta_field_row(const carekv_arena& A, long pg_base, int p, bool ok, int f) {
  const uint32_t pp = ok ? (uint32_t)p : 0u;
  const bool in_ks = f >= 2 && f < 2 + NCG, in_vs = f >= 6 && f < 6 + kVtb;
  const uint32_t fk = in_ks ? (uint32_t)(f - 2) : 0u, fv = in_vs ? (uint32_t)(f - 6) : 0u;
  // 32-bit byte offsets from uniform bases: SGPR-base + VGPR-offset loads
  const int vk = ld_off<int>(A.k_slot + pg_base * NCG, (pp * NCG + fk) * 4u);
  const int vv = ld_off<int>(A.v_slot + pg_base * kVtb, (pp * kVtb + fv) * 4u);
  const int vn = ld_off<int>(A.valid + pg_base, pp * 4u);
  int v16 = 0;
  if constexpr (SM == 1) {
    const int mk = (int)ld_off<uint16_t>(A.kmaster + pg_base, pp * 2u);
    const int mv = (int)ld_off<uint16_t>(A.vmaster + pg_base, pp * 2u);
    v16 = f == 11 ? mv : mk;
  }
  const int v8 = (int)ld_off<int8_t>(A.has_meta + pg_base, pp);
  int v = 0;
  if (f == 0) v = vn;
  if (in_ks) v = vk;
  if (in_vs) v = vv;
  if (f == 1) v = v8;
  if (f == 10 || f == 11) v = v16;
  return ok ? v : 0;
}

// Field f of page pg (the layout of meta_field_row) in two steps:
// meta_word_load issues one 32-bit load of the
// aligned word that holds field f of page pg (the 16-bit masters and the
// 8-bit has_meta are read through the aligned word holding them; such a word
// lies in the same mapped page as the field), and meta_word_field extracts
// the field where it is used.  A prefetch that selects among several loads
// at once waits for all of them right behind the loads; one raw word waits
// only where its field is first needed.
template <int NCG, int SM>
__device__ __forceinline__ uint32_t meta_word_load(const carekv_arena& A, long pg, int f) {
  const bool in_ks = f >= 2 && f < 2 + NCG, in_vs = f >= 6 && f < 6 + kVtb;
  const char* p;
  if (in_ks) p = reinterpret_cast<const char*>(A.k_slot + pg * NCG + (f - 2));
  else if (in_vs) p = reinterpret_cast<const char*>(A.v_slot + pg * kVtb + (f - 6));
  else if (f == 1) p = reinterpret_cast<const char*>(A.has_meta + pg);
  else if (SM == 1 && f == 10) p = reinterpret_cast<const char*>(A.kmaster + pg);
  else if (SM == 1 && f == 11) p = reinterpret_cast<const char*>(A.vmaster + pg);
  else p = reinterpret_cast<const char*>(A.valid + pg);  // field 0; other fields drop the word
  // aligned by pointer arithmetic on p, which keeps its (global) address space
  return *reinterpret_cast<const uint32_t*>(p - (reinterpret_cast<uintptr_t>(p) & 3u));
}
template <int NCG, int SM>
__device__ __forceinline__ int meta_word_field(const carekv_arena& A, uint32_t w, long pg, int f) {
  const bool in_ks = f >= 2 && f < 2 + NCG, in_vs = f >= 6 && f < 6 + kVtb;
  if (f == 0 || in_ks || in_vs) return (int)w;
  if (f == 1) return (int)(int8_t)(w >> (8u * (uint32_t)(reinterpret_cast<uintptr_t>(A.has_meta + pg) & 3u)));
  if (SM == 1 && (f == 10 || f == 11)) {
    const uint16_t* m = f == 10 ? A.kmaster + pg : A.vmaster + pg;
    return (int)((w >> (8u * (uint32_t)(reinterpret_cast<uintptr_t>(m) & 2u))) & 0xffffu);
  }
  return 0;
}

// ---------------------------------------------------------------- 4x4x4 PV
// O[q][slot] += sum_m P[q][g + 4m] V_tile[g + 4m][slot], m = 0..3 (token
// group g of a 16-row tile: rows g, g+4, g+8, g+12), on
// v_mfma_f32_4x4x4_16b_f16 with A = V^T (block b = slots 4b..4b+3 of a
// 64-slot half) and B = P (4 query heads):
//   * the A operand comes from the token-major tile through the transpose
//     load: source lane s of 16-lane group G reads row g + 4(s/4), slots
//     16G + 4(s%4) .. +3, and lane r of the group receives slots 16G + r of
//     rows g, g+4, g+8, g+12.  With the row stride of D/2 + 4 words, the 4
//     rows 4 apart sit 16 banks apart, so each half-wave's 32 reads hit 64
//     distinct banks (rows 1 apart would overlap);
//   * p01/p23 hold P[query lane % 4][tokens g, g+4, g+8, g+12] as fp16 pairs.
// Lane l accumulates O[query l % 4][slots 64h + 4(l/4) .. +3] in acc[h].
template <int D, int BITS>
__device__ __forceinline__ void pv4_group(const uint32_t* vt, int g, uint32_t p01, uint32_t p23, float4_t* acc,
                                          int lane) {
  using G = PageGeom<D, BITS>;
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  half4_t bq;
  __builtin_memcpy(&bq, &p01, 4);
  __builtin_memcpy(reinterpret_cast<char*>(&bq) + 4, &p23, 4);
  const int s = lane & 15, g16 = lane >> 4;
  const __attribute__((address_space(3))) char* base = (const __attribute__((address_space(3))) char*)vt +
                                                       ((g + 4 * (s >> 2)) * G::VROW) * 4 + (16 * g16 + 4 * (s & 3)) * 2;
#pragma unroll
  for (int h = 0; h < D / 64; ++h) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + 128 * h));
    half4_t av;
    __builtin_memcpy(&av, &v, 8);
    acc[h] = mfma4x4(av, bq, acc[h]);
  }
}

// Weights of a 4-page window for the 4x4x4 PV, staged per wave in LDS.  The
// S-layout lane 16*pi + 4*j + q (page pi, tokens 4j..4j+3, query q):
//   * pw_store puts its 4 fp16 weights at pw[pi][q][j] (token groups of 4
//     consecutive tokens);
//   * pw_store_strided puts weight i at pw[pi][q][i][j], so that entry
//     [pi][q][g] holds tokens g, g+4, g+8, g+12 (the token groups of
//     pv4_group).
// A lane then reads the 4 groups of a page for its own query with two
// 16-byte loads (pw_load).
__device__ __forceinline__ void pw_store(uint2* pw, uint32_t w01, uint32_t w23, int lane) {
  pw[((lane >> 4) * 4 + (lane & 3)) * 4 + ((lane >> 2) & 3)] = make_uint2(w01, w23);
}
__device__ __forceinline__ void pw_store_strided(uint2* pw, uint32_t w01, uint32_t w23, int lane) {
  uint16_t* h = reinterpret_cast<uint16_t*>(pw) + ((lane >> 4) * 4 + (lane & 3)) * 16 + ((lane >> 2) & 3);
  h[0] = (uint16_t)w01;
  h[4] = (uint16_t)(w01 >> 16);
  h[8] = (uint16_t)w23;
  h[12] = (uint16_t)(w23 >> 16);
}
__device__ __forceinline__ void pw_load(const uint2* pw, int pi, int q, uint2 (&p)[4]) {
  const uint4* s = reinterpret_cast<const uint4*>(pw + (pi * 4 + q) * 4);
  const uint4 a = s[0], b = s[1];
  p[0] = make_uint2(a.x, a.y);
  p[1] = make_uint2(a.z, a.w);
  p[2] = make_uint2(b.x, b.y);
  p[3] = make_uint2(b.z, b.w);
}

// Dim of slot s (slot order of the base pair schedule, chunks of CH).
template <int D, int BITS>
__device__ __forceinline__ int slot_dim(int slot) {
  using G = PageGeom<D, BITS>;
  return (slot / G::CH) * G::CH + G::PB::T.slot_code[slot % G::CH];
}

// Field offset o of slot s in code_pair_sub form (its value is u * 2^(o-24)).
template <int D, int BITS>
__device__ __forceinline__ int slot_off(int slot) {
  using G = PageGeom<D, BITS>;
  const int r = slot % G::CH, i = r >> 1;
  return (r & 1) ? G::PB::T.bo[i] : G::PB::T.ao[i];
}

// ---------------------------------------------------------------- 4x4x4 PV on raw V codes
// The V scales (one per token and 32-dim group) move from the codes into
// the weights: P'[q][t][G] = half(P[q][t] * s_V[t][G]), so the V tile holds
// the codes in code_pair_sub form and needs one bitop3 per pair.  In a PV
// step over the 64-slot half h, lanes 0-31 cover group 2h and lanes 32-63
// group 2h + 1 (slots 64h .. 64h+31 and 64h+32 .. 64h+63 are the chunks of
// one group each at D = 128, and of half a group each at D = 64).
//
// Weights per wave in LDS, fp16 [page][G][query][16]: entry i*4 + m holds
// token 4m + i, so that the 4 halves of [g*4 .. g*4+3] are the tokens g,
// g+4, g+8, g+12 of pv4_group.  The S-layout lane 16*pi + 4*j + q (tokens
// 4j..4j+3 of page pi, query q) writes its 4 weights of group G.
template <int NCG>
__device__ __forceinline__ void pwg_store(uint16_t* pw, int G, uint32_t w01, uint32_t w23, int lane) {
  uint16_t* h = pw + (((lane >> 4) * NCG + G) * 4 + (lane & 3)) * 16 + ((lane >> 2) & 3);
  h[0] = (uint16_t)w01;
  h[4] = (uint16_t)(w01 >> 16);
  h[8] = (uint16_t)w23;
  h[12] = (uint16_t)(w23 >> 16);
}
template <int NCG>
__device__ __forceinline__ void pwg_load(const uint16_t* pw, int pi, int G, int q, uint2 (&p)[4]) {
  const uint4* s = reinterpret_cast<const uint4*>(pw + ((pi * NCG + G) * 4 + q) * 16);
  const uint4 a = s[0], b = s[1];
  p[0] = make_uint2(a.x, a.y);
  p[1] = make_uint2(a.z, a.w);
  p[2] = make_uint2(b.x, b.y);
  p[3] = make_uint2(b.z, b.w);
}

// One PV step of token group g over the 64-slot half h (the layout of
// pv4_group) with the weights p01/p23 of the lane's group.
template <int D, int BITS>
__device__ __forceinline__ void pv4_step(const uint32_t* vt, int g, int h, uint32_t p01, uint32_t p23, float4_t& acc,
                                         int lane) {
  using G = PageGeom<D, BITS>;
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;
  half4_t bq;
  __builtin_memcpy(&bq, &p01, 4);
  __builtin_memcpy(reinterpret_cast<char*>(&bq) + 4, &p23, 4);
  const int s = lane & 15, g16 = lane >> 4;
  const __attribute__((address_space(3))) char* base = (const __attribute__((address_space(3))) char*)vt +
                                                       ((g + 4 * (s >> 2)) * G::VROW) * 4 + (16 * g16 + 4 * (s & 3)) * 2 +
                                                       128 * h;
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)base);
  half4_t av;
  __builtin_memcpy(&av, &v, 8);
  acc = mfma4x4(av, bq, acc);
}

// merge4_waves for accumulators over raw codes: slot s of the lane's query
// is acc * 2^(24 - o(s)) - 2^(BITS-1) * wsum, wsum = the lane's group's
// weight sum over the split (bias[h] for the half h).
template <int D, int BITS>
__device__ __forceinline__ void merge4_waves_raw(float* so, float (*s_m)[4], float (*s_l)[4], float m_run, float l_run,
                                                 const float4_t* acc, const float* bias, int w, int lane, int GQ,
                                                 float* po, float* pml) {
  constexpr float top = (float)(1 << (BITS - 1));
  __syncthreads();
  if (lane < 4) { s_m[w][lane] = m_run; s_l[w][lane] = l_run; }
  const int q = lane & 3, b = lane >> 2;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = 64 * h + 4 * b + i;
      so[(w * 4 + q) * D + slot_dim<D, BITS>(slot)] =
          fmaf(acc[h][i], __builtin_ldexpf(1.0f, 24 - slot_off<D, BITS>(slot)), -top * bias[h]);
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < GQ * D; idx += blockDim.x) {
    const int qq = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][qq]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float f = __builtin_amdgcn_exp2f(s_m[ww][qq] - M);
        L += s_l[ww][qq] * f;
        O += so[(ww * 4 + qq) * D + d] * f;
      }
    }
    po[qq * D + d] = O;
    if (d == 0) { pml[qq * 2] = M; pml[qq * 2 + 1] = L; }
  }
}

// merge_waves for the 4x4x4 PV layout (lane l: query l % 4, slots
// 64h + 4(l/4) + i): so holds [4 waves][4 queries][D] fp32.
template <int D, int BITS>
__device__ __forceinline__ void merge4_waves(float* so, float (*s_m)[4], float (*s_l)[4], float m_run, float l_run,
                                             const float4_t* acc, int w, int lane, int GQ, float* po, float* pml) {
  __syncthreads();
  if (lane < 4) { s_m[w][lane] = m_run; s_l[w][lane] = l_run; }
  const int q = lane & 3, b = lane >> 2;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[(w * 4 + q) * D + slot_dim<D, BITS>(64 * h + 4 * b + i)] = acc[h][i];
  __syncthreads();
  for (int idx = threadIdx.x; idx < GQ * D; idx += blockDim.x) {
    const int qq = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, s_m[ww][qq]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float f = __builtin_amdgcn_exp2f(s_m[ww][qq] - M);
        L += s_l[ww][qq] * f;
        O += so[(ww * 4 + qq) * D + d] * f;
      }
    }
    po[qq * D + d] = O;
    if (d == 0) { pml[qq * 2] = M; pml[qq * 2 + 1] = L; }
  }
}

// sum_waves for the 4x4x4 PV layout: out[q][d] = sum over the 4 waves.
template <int D, int BITS>
__device__ __forceinline__ void sum4_waves(float* so, const float4_t* acc, int w, int lane, int GQ, float* out) {
  __syncthreads();
  const int q = lane & 3, b = lane >> 2;
#pragma unroll
  for (int h = 0; h < D / 64; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) so[(w * 4 + q) * D + slot_dim<D, BITS>(64 * h + 4 * b + i)] = acc[h][i];
  __syncthreads();
  for (int idx = threadIdx.x; idx < GQ * D; idx += blockDim.x) {
    const int qq = idx / D, d = idx % D;
    out[qq * D + d] = ((so[qq * D + d] + so[(4 + qq) * D + d]) + so[(8 + qq) * D + d]) + so[(12 + qq) * D + d];
  }
}

}  // namespace carekv
