// Prefill attention over dequantised K/V (CAREKVLayer._causal_attention_pure,
// layer.py:935-972) on v_mfma_f32_16x16x32_f16, flash style: the (T, T)
// score and weight matrices are never materialised; the kernel returns O and,
// optionally, the per-row log-sum-exp from which any weight can be rebuilt.
//
// One work-group per (block of 128 queries, query head, sequence), 4 waves of
// 32 queries, on a one-dimensional grid whose order starts the longest
// (latest) query blocks of every (sequence, head) first.  K and V tiles of 32
// tokens are staged in LDS (double buffered, one barrier per tile; the next
// tile's global loads are in flight while the current one is used); at
// D = 128, 160 VGPRs and 35 KB of LDS, three work-groups share a CU:
//   * S^T = K_hat Q^T: A = K tile rows (one 16-byte LDS read per lane and
//     32-dim step), B = Q^T held in registers; lane l receives the scores of
//     tokens 16tt + 4(l/16) + i for query l % 16 of a 16-query sub-block;
//   * the online softmax runs per query column in fp32 on base-2 logits
//     (scores scaled by log2(e)/sqrt(D) after the fp32 product, as the
//     reference divides the fp32 product by sqrt(D));
//   * O^T += V_hat^T P^T: the weights are already in the B layout (the 8 k
//     values of a lane are tokens 4(l/16) + i of two 16-token tiles), and
//     the A operand V_hat^T comes from the token-major V tile through the
//     gfx950 transpose load ds_read_b64_tr_b16 for the same token order.
// The K tile rows are padded to 2D + 16 bytes and the V tile rows to 2D + 32
// bytes, so that each group of consecutive lanes of either LDS read pattern
// touches every bank once.
#include <cmath>

#include "decode_page.h"
#include "host_util.h"

namespace carekv {

struct PrefillArgs {
  const uint16_t* q;  // [B][Hq][T][D]
  const uint16_t* k;  // [B][Hkv][T][D]
  const uint16_t* v;
  uint16_t* out;      // [B][Hq][T][D]
  float* lse;         // [B][Hq][T] natural log-sum-exp of the scaled scores, or null
  int B, Hq, Hkv, T, causal;
  float sm_log2;      // sm_scale * log2(e)
};

template <int D>
__global__ __launch_bounds__(256, 3) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int KT = 32;              // tokens per K/V tile
  constexpr int TT = KT / 16, NU = KT / 32;
  constexpr int QB = 128;             // queries per work-group
  constexpr int KRS = 2 * D + 16;     // K tile row stride, bytes
  constexpr int VRS = 2 * D + 32;     // V tile row stride, bytes
  constexpr int KS = D / 32;          // 32-dim steps of the score product
  constexpr int DT = D / 16;          // 16-dim output tiles
  constexpr int KBUF = KT * KRS, VBUF = KT * VRS, BUF = KBUF + VBUF;
  constexpr int CHR = D / 8;          // 16-byte chunks per row
  constexpr int NCH = 2 * KT * CHR / 256;  // chunks a thread stages per tile
  __shared__ __align__(16) char lds[2 * BUF];
  typedef short short4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) short4_t lds_short4;

  // the longest (latest) query blocks of every (sequence, head) start first
  const int nhb = a.Hq * a.B, nqb = gridDim.x / nhb;
  const int qblk = nqb - 1 - (int)blockIdx.x / nhb, hb = (int)blockIdx.x % nhb;
  const int h = hb % a.Hq, b = hb / a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int T = a.T;
  const int q0 = qblk * QB, qw0 = q0 + 32 * w;
  const uint32_t span = (uint32_t)T * D * 2;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + ((long)b * a.Hq + h) * T * D, span);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k + ((long)b * a.Hkv + hk) * T * D, span);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v + ((long)b * a.Hkv + hk) * T * D, span);

  // Q^T operands: sub-block qb, step s -> query qw0 + 16 qb + c16, dims 32s + 8g ..
  half8_t qf[2][KS];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t qi = (uint32_t)(qw0 + 16 * qb + c16);
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rq, (qi * D + 32 * s + 8 * g) * 2, 0, 0);
      __builtin_memcpy(&qf[qb][s], &v, 16);
    }

  const int q_last = min(q0 + QB, T) - 1;
  const int nt = a.causal ? q_last / KT + 1 : (T + KT - 1) / KT;

  // staging: chunk c = threadIdx.x + 256 k -> tensor c / (KT CHR) (K, V), row, 16-byte column
  uint32_t stg[NCH][4];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = threadIdx.x + 256 * k;
      const int rc = c % (KT * CHR), row = rc / CHR, col = rc % CHR;
      const uint32_t off = ((uint32_t)(j * KT + row) * D + col * 8) * 2;
      // chunks 0 .. KT*CHR-1 are K, the rest V: with 256 threads that is
      // k < NCH / 2, known at compile time (a per-lane choice of resource
      // would make every load a waterfall loop)
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

  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  float4_t o[2][DT];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[qb][dt] = float4_t{0.f, 0.f, 0.f, 0.f};

  load_tile(0);
  store_tile(0);
  __syncthreads();
  if (nt > 1) load_tile(1);

  for (int j = 0; j < nt; ++j) {
    const char* kb = lds + (j & 1) * BUF;
    const char* vb = kb + KBUF;
    const int t0 = j * KT;
    if (!a.causal || t0 <= qw0 + 31) {  // some query of the wave sees this tile
      // ---- S^T = K_hat Q^T (raised wave priority over the MFMA blocks: a wave
      // with products to issue goes before the CU's other waves' softmax)
      __builtin_amdgcn_s_setprio(1);
      float4_t s[TT][2];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        s[tt][0] = float4_t{0.f, 0.f, 0.f, 0.f};
        s[tt][1] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          half8_t ak;
          *reinterpret_cast<uint4*>(&ak) = *reinterpret_cast<const uint4*>(kb + (16 * tt + c16) * KRS + (32 * ks + 8 * g) * 2);
          s[tt][0] = mfma16x32(ak, qf[0][ks], s[tt][0]);
          s[tt][1] = mfma16x32(ak, qf[1][ks], s[tt][1]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      // ---- mask (the wave's diagonal and the end of the sequence), then
      // the base-2 logits x = s * log2(e)/sqrt(D) folded into the exponent:
      // max x = c * max s for c > 0 (rounding is monotone), and
      // exp2(x - m) is taken as exp2(fma(s, c, -m))
      const bool edge = (a.causal && t0 + KT - 1 > qw0) || t0 + KT > T;
      const float c = a.sm_log2;
      float p[TT][2][4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qi = qw0 + 16 * qb + c16;
        if (edge) {
          // token 16 tt + i of the lane's rows is t0 + 4g + 16 tt + i; the
          // limits pass through an empty asm so that the compares stay on
          // this branch (most tiles are not edge tiles)
          int lim_t = T - t0 - 4 * g, lim_q = a.causal ? qi - t0 - 4 * g : 0x3fffffff;
          asm volatile("" : "+v"(lim_t), "+v"(lim_q));
#pragma unroll
          for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int o = 16 * tt + i;
              if (o >= lim_t || o > lim_q) s[tt][qb][i] = -INFINITY;
            }
        }
        // a chain of three-operand maxima over the lane's 16 scores
        float mx = s[0][qb][0];
#pragma unroll
        for (int k = 1; k < 4 * TT; k += 2) {
          const int k2 = k + 1 < 4 * TT ? k + 1 : k;
          mx = fmaxf(fmaxf(mx, s[k / 4][qb][k % 4]), s[k2 / 4][qb][k2 % 4]);
        }
        mx = pair32_max(pair16_max(mx)) * c;
        const float m_new = fmaxf(m_run[qb], mx);  // finite: token 0 is visible to every query
        const float f = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
        m_run[qb] = m_new;
        float ls = 0.f;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(fmaf(s[tt][qb][i], c, -m_new));
            p[tt][qb][i] = e;
            ls += e;
          }
        l_run[qb] = l_run[qb] * f + ls;  // this lane's tokens; summed over the lane groups at the end
        if (__builtin_expect(__any(f != 1.f), 0)) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[qb][dt] *= f;
        }
      }
      __builtin_amdgcn_s_setprio(1);
      // ---- O^T += V_hat^T P^T, 32 tokens per step
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        half8_t bp[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          bp[qb] = half8_t{(_Float16)p[2 * u][qb][0], (_Float16)p[2 * u][qb][1], (_Float16)p[2 * u][qb][2],
                           (_Float16)p[2 * u][qb][3], (_Float16)p[2 * u + 1][qb][0], (_Float16)p[2 * u + 1][qb][1],
                           (_Float16)p[2 * u + 1][qb][2], (_Float16)p[2 * u + 1][qb][3]};
        // source lane c16 of group g reads row 32u + 4g + c16/4 (and +16), dims 16dt + 4(c16%4) ..
        const __attribute__((address_space(3))) char* vrow =
            (const __attribute__((address_space(3))) char*)vb + (32 * u + 4 * g + (c16 >> 2)) * VRS + (c16 & 3) * 8;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const short4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrow + 32 * dt));
          const short4_t v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vrow + 16 * VRS + 32 * dt));
          half8_t av;
          __builtin_memcpy(&av, &v1, 8);
          __builtin_memcpy(reinterpret_cast<char*>(&av) + 8, &v2, 8);
          o[0][dt] = mfma16x32(av, bp[0], o[0][dt]);
          o[1][dt] = mfma16x32(av, bp[1], o[1][dt]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (j + 1 < nt) store_tile((j + 1) & 1);
    if (j + 2 < nt) load_tile(j + 2);
    __syncthreads();
  }

  // ---- normalise and write (lane: query qw0 + 16qb + c16, dims 16dt + 4g ..)
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float lt = pair32_sum(pair16_sum(l_run[qb]));
    const float inv = 1.f / lt;
    const int qi = qw0 + 16 * qb + c16;
    if (qi < T) {
      uint16_t* dst = a.out + (((long)b * a.Hq + h) * T + qi) * D + 4 * g;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint32_t lo = (uint32_t)f2h(o[qb][dt][0] * inv) | ((uint32_t)f2h(o[qb][dt][1] * inv) << 16);
        const uint32_t hi = (uint32_t)f2h(o[qb][dt][2] * inv) | ((uint32_t)f2h(o[qb][dt][3] * inv) << 16);
        *reinterpret_cast<uint2*>(dst + 16 * dt) = make_uint2(lo, hi);
      }
      if (a.lse && g == 0) a.lse[((long)b * a.Hq + h) * T + qi] = (m_run[qb] + __log2f(lt)) * 0.69314718f;
    }
  }
}

// x_hat = half(code * scale) per group of 32 (quantizer.py:67-82): the
// product of an int8 code and an fp16 scale is exact in fp32 and is rounded
// once to fp16.
__global__ void dequantize_rows_kernel(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scale,
                                       long n, int D, uint16_t* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const long r = i / D;
  const int d = (int)(i % D);
  out[i] = f2h((float)codes[i] * h2f(scale[r * (D / 32) + d / 32]));
}

// carekv_eval prefill correction (CAREKVLayer._apply_sparse_prefill_correction_eval,
// layer.py:363-456): one work-group per (row t, query head, sequence).
//   0. the row's softmax in fp32 over x_j = q.K_hat_j / sqrt(D), j <= t
//      (max, then the sum of exp(x - max); layer.py:963), as the base
//      weights a_j = half(exp(x_j - max) / sum) of the reference;
//   1. every token j <= t of the row, 16 lanes a token (D/16 dims a lane):
//      q.K_hat_j, q.r_k, ||r_v||^2, ||V_hat_j - o||^2 with r_k =
//      half(K - K_hat), r_v = half(V - V_hat) (layer.py:770-775); a_j; the V
//      and K scores to LDS;
//   2. the final scores (kind, per-kind mean normalisation);
//   3. the k-th largest score by a bitwise search over the (non-negative)
//      float bits, then the selected tokens in index order (ties at the k-th
//      value to the lower indices);
//   4. dO_V and dO_K over the selected tokens, with the terms recomputed by
//      the same code as in 1 (same values), summed over the waves in LDS.
constexpr int kEvalMaxT = 8192;

struct EvalArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* kh;
  const uint16_t* vh;
  const uint16_t* o;
  uint16_t* out;
  int32_t* diag;
  int B, Hq, Hkv, T, diag_cap, min_res, kind, v_norm, normalize;
  double ratio;
  float k_corr, inv_sqrt_d, sqrt_d;
};

template <int D>
__global__ __launch_bounds__(256) void prefill_eval_kernel(EvalArgs a) {
  constexpr int PL = D / 16;  // dims a lane holds of its token
  // sized at launch to the prompt (2 T words), so that short prompts fit
  // more work-groups per CU: [T] V scores, then the final scores; [T] K
  // scores (float bits), then the selected tokens
  extern __shared__ float s_dyn[];
  float* const s_v = s_dyn;
  int* const s_k = reinterpret_cast<int*>(s_dyn + a.T);
  __shared__ float s_red[4][4];
  __shared__ int s_cnt[2][256];
  __shared__ float s_acc[4][2][D];
  // a one-dimensional grid, the latest (longest) rows of every (sequence, head) first
  const int nhb = a.Hq * a.B, hb = (int)blockIdx.x % nhb;
  const int t = a.T - 1 - (int)blockIdx.x / nhb, h = hb % a.Hq, b = hb / a.Hq;
  const int hk = h / (a.Hq / a.Hkv);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane & 15, slot = lane >> 4;  // dims c*PL.., token slot of the wave
  const int n = t + 1;
  const long rowoff = (((long)b * a.Hq + h) * a.T + t) * D;
  const long kvbase = ((long)b * a.Hkv + hk) * a.T * D;
  float qf[PL], of[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    qf[i] = h2f(a.q[rowoff + c * PL + i]);
    of[i] = h2f(a.o[rowoff + c * PL + i]);
  }

  // the terms of token j (every lane of the 16-lane group ends with the totals)
  auto terms = [&](int j, float& sq, float& qd, float& rvn2, float& vd2, float (&rv)[PL], float (&vh)[PL]) {
    const long r = kvbase + (long)j * D + c * PL;
    sq = qd = rvn2 = vd2 = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const float kk = h2f(a.k[r + i]), kh = h2f(a.kh[r + i]);
      const float vv = h2f(a.v[r + i]);
      vh[i] = h2f(a.vh[r + i]);
      sq = fmaf(qf[i], kh, sq);
      const float rk = (float)(_Float16)(kk - kh);
      qd = fmaf(qf[i], rk, qd);
      rv[i] = (float)(_Float16)(vv - vh[i]);
      rvn2 = fmaf(rv[i], rv[i], rvn2);
      const float dv = vh[i] - of[i];
      vd2 = fmaf(dv, dv, vd2);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      sq += __shfl_xor(sq, o, 64);
      qd += __shfl_xor(qd, o, 64);
      rvn2 += __shfl_xor(rvn2, o, 64);
      vd2 += __shfl_xor(vd2, o, 64);
    }
  };

  // ---- 0. the row's fp32 softmax: max and sum of exp(x - max), x = q.K_hat / sqrt(D)
  float mx = -INFINITY;
  for (int j0 = 0; j0 < n; j0 += 16) {
    const int j = j0 + 4 * w + slot;
    const bool ok = j < n;
    const long r = kvbase + (long)(ok ? j : 0) * D + c * PL;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i) sq = fmaf(qf[i], h2f(a.kh[r + i]), sq);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o, 64);
    if (ok && c == 0) {
      const float x = sq / a.sqrt_d;
      s_v[j] = x;
      mx = fmaxf(mx, x);
    }
  }
  mx = wave_max(mx);
  if (lane == 0) s_red[0][w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
  float es = 0.f;
  for (int j = tid; j < n; j += 256) es += expf(s_v[j] - mx);
  es = wave_sum(es);
  if (lane == 0) s_red[1][w] = es;
  __syncthreads();
  const float den = ((s_red[1][0] + s_red[1][1]) + s_red[1][2]) + s_red[1][3];
  // the fp16 base weight (softmax in fp32, cast to fp16)
  auto weight = [&](float sq) { return (float)(_Float16)(expf(sq / a.sqrt_d - mx) / den); };

  // ---- 1. token scores
  float vsum = 0.f, ksum = 0.f;
  for (int j0 = 0; j0 < n; j0 += 16) {
    const int j = j0 + 4 * w + slot;
    const bool ok = j < n;
    float sq, qd, rvn2, vd2, rv[PL], vh[PL];
    terms(ok ? j : 0, sq, qd, rvn2, vd2, rv, vh);
    if (ok && c == 0) {
      const float aw = weight(sq);
      const float vdiff = sqrtf(vd2), qdot = qd * a.inv_sqrt_d;
      float vs = aw * sqrtf(rvn2);
      if (!a.v_norm) vs = vs * vdiff;
      const float ks = aw * fabsf(qdot) * vdiff;
      s_v[j] = vs;
      s_k[j] = __float_as_int(ks);
      vsum += fabsf(vs);
      ksum += fabsf(ks);
    }
  }
  vsum = wave_sum(vsum);
  ksum = wave_sum(ksum);
  if (lane == 0) { s_red[2][w] = vsum; s_red[3][w] = ksum; }
  __syncthreads();
  // ---- 2. final scores
  {
    const float vm = fmaxf((((s_red[2][0] + s_red[2][1]) + s_red[2][2]) + s_red[2][3]) / (float)n, 1e-8f);
    const float km = fmaxf((((s_red[3][0] + s_red[3][1]) + s_red[3][2]) + s_red[3][3]) / (float)n, 1e-8f);
    for (int j = tid; j < n; j += 256) {
      const float vs = s_v[j], ks = __int_as_float(s_k[j]);
      s_v[j] = a.kind == 2 ? vs : a.kind == 1 ? ks : (a.normalize ? vs / vm + ks / km : vs + ks);
    }
  }
  __syncthreads();
  // int(n * ratio) (layer.py:397); a ratio of 1 or more keeps all n, so the
  // conversion only ever sees values below n
  int K = a.ratio >= 1.0 ? n : (int)((double)n * a.ratio);
  K = min(max(a.min_res, K), n);
  // block sum of an int (two barriers)
  auto block_count = [&](int x, int which) -> int {
    x = (int)wave_sum((float)x);
    if (lane == 0) s_cnt[which][w] = x;
    __syncthreads();
    const int tot = s_cnt[which][0] + s_cnt[which][1] + s_cnt[which][2] + s_cnt[which][3];
    __syncthreads();
    return tot;
  };
  // ---- 3. the k-th largest score and the selected tokens in index order
  int nsel = 0;
  if (K > 0) {
    uint32_t tau = 0u;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = tau | (1u << bit);
      int cnt = 0;
      for (int j = tid; j < n; j += 256) cnt += __float_as_uint(s_v[j]) >= cand;
      if (block_count(cnt, 0) >= K) tau = cand;
    }
    const int L = (n + 255) / 256, j0 = tid * L, j1 = min(j0 + L, n);
    int gt = 0, eq = 0;
    for (int j = j0; j < j1; ++j) {
      const uint32_t x = __float_as_uint(s_v[j]);
      gt += x > tau;
      eq += x == tau;
    }
    const int need_eq = K - block_count(gt, 0);
    s_cnt[0][tid] = eq;
    __syncthreads();
    if (tid == 0) {  // exclusive scans: equal tokens before each chunk, then selected tokens
      int acc = 0;
      for (int i = 0; i < 256; ++i) { const int e = s_cnt[0][i]; s_cnt[0][i] = acc; acc += e; }
    }
    __syncthreads();
    const int eq_take = min(max(need_eq - s_cnt[0][tid], 0), eq);
    s_cnt[1][tid] = gt + eq_take;
    __syncthreads();
    if (tid == 0) {
      int acc = 0;
      for (int i = 0; i < 256; ++i) { const int e = s_cnt[1][i]; s_cnt[1][i] = acc; acc += e; }
    }
    __syncthreads();
    int pos = s_cnt[1][tid], taken = 0;
    for (int j = j0; j < j1; ++j) {
      const uint32_t x = __float_as_uint(s_v[j]);
      if (x > tau || (x == tau && taken < eq_take)) {
        taken += x == tau;
        s_k[pos++] = j;  // the K scores are consumed
      }
    }
    nsel = K;
    __syncthreads();
  }
  // ---- 4. corrections over the selected tokens
  float dv[PL], dk[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) dv[i] = dk[i] = 0.f;
  for (int i0 = 0; i0 < nsel; i0 += 16) {
    const int i = i0 + 4 * w + slot;
    const bool ok = i < nsel;
    const int j = s_k[ok ? i : 0];
    float sq, qd, rvn2, vd2, rv[PL], vh[PL];
    terms(j, sq, qd, rvn2, vd2, rv, vh);
    if (ok) {
      const float aw = weight(sq);
      const float qc = fminf(fmaxf(qd * a.inv_sqrt_d, -2.f), 2.f);
#pragma unroll
      for (int p = 0; p < PL; ++p) {
        dv[p] += aw * rv[p];
        dk[p] += (aw * qc) * (vh[p] - of[p]);
      }
    }
  }
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    dv[p] += __shfl_xor(dv[p], 16, 64);
    dv[p] += __shfl_xor(dv[p], 32, 64);
    dk[p] += __shfl_xor(dk[p], 16, 64);
    dk[p] += __shfl_xor(dk[p], 32, 64);
  }
  if (slot == 0) {
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      s_acc[w][0][c * PL + p] = dv[p];
      s_acc[w][1][c * PL + p] = dk[p];
    }
  }
  __syncthreads();
  for (int d = tid; d < D; d += 256) {
    const float o = h2f(a.o[rowoff + d]);
    const float tv = a.kind == 1 ? 0.f : ((s_acc[0][0][d] + s_acc[1][0][d]) + s_acc[2][0][d]) + s_acc[3][0][d];
    const float tk = a.kind == 2 ? 0.f : ((s_acc[0][1][d] + s_acc[1][1][d]) + s_acc[2][1][d]) + s_acc[3][1][d];
    a.out[rowoff + d] = f2h((o + tv) + a.k_corr * tk);
  }
  if (a.diag) {
    int32_t* dg = a.diag + (((long)b * a.Hq + h) * a.T + t) * a.diag_cap;
    for (int i = tid; i < a.diag_cap; i += 256) dg[i] = i < nsel ? s_k[i] : -1;
  }
}

}  // namespace carekv

using namespace carekv;

extern "C" int carekv_prefill_eval(const carekv_prefill_eval_params* p, const uint16_t* q, const uint16_t* k,
                                   const uint16_t* v, const uint16_t* k_hat, const uint16_t* v_hat,
                                   const uint16_t* o_base, uint16_t* out, int32_t* diag, void* stream) {
  CAREKV_REQUIRE(p && q && k && v && k_hat && v_hat && o_base && out, "null argument");
  CAREKV_REQUIRE(p->head_dim == 64 || p->head_dim == 128, "head_dim must be 64 or 128");
  CAREKV_REQUIRE(p->batch > 0 && p->n_heads > 0 && p->n_kv_heads > 0 && p->n_heads % p->n_kv_heads == 0,
                 "batch and head counts must be positive, n_heads a multiple of n_kv_heads");
  CAREKV_REQUIRE(p->seq_len > 0 && p->seq_len <= kEvalMaxT, "seq_len must be in 1..8192");
  // Python's int(n * ratio) raises on an infinite or NaN product (layer.py:397)
  CAREKV_REQUIRE(std::isfinite(p->ratio), "ratio must be finite");
  CAREKV_REQUIRE(p->ratio >= 0.0 && p->min_residuals >= 0, "ratio and min_residuals must be non-negative");
  CAREKV_REQUIRE(p->kind >= 0 && p->kind <= 2, "kind must be 0 (both), 1 (k) or 2 (v)");
  CAREKV_REQUIRE(!diag || p->diag_cap > 0, "diag needs diag_cap > 0");
  EvalArgs a{};
  a.q = q; a.k = k; a.v = v; a.kh = k_hat; a.vh = v_hat; a.o = o_base; a.out = out; a.diag = diag;
  a.B = p->batch; a.Hq = p->n_heads; a.Hkv = p->n_kv_heads; a.T = p->seq_len; a.diag_cap = diag ? p->diag_cap : 0;
  a.min_res = p->min_residuals; a.kind = p->kind; a.v_norm = p->v_score_norm != 0; a.normalize = p->normalize != 0;
  a.ratio = p->ratio; a.k_corr = p->k_corr_scale;
  a.sqrt_d = (float)std::sqrt((double)p->head_dim);
  a.inv_sqrt_d = (float)(1.0 / std::sqrt((double)p->head_dim));
  const long nblk = (long)p->seq_len * p->n_heads * p->batch;
  CAREKV_REQUIRE(nblk < (1L << 31), "too many (row, head, sequence) work-groups");
  const dim3 grid((unsigned)nblk);
  const size_t shmem = (size_t)p->seq_len * 2 * sizeof(float);
  hipStream_t s = (hipStream_t)stream;
  if (p->head_dim == 128) hipLaunchKernelGGL(prefill_eval_kernel<128>, grid, dim3(256), shmem, s, a);
  else hipLaunchKernelGGL(prefill_eval_kernel<64>, grid, dim3(256), shmem, s, a);
  CAREKV_CHECK_LAUNCH("prefill_eval");
  return CAREKV_OK;
}

extern "C" int carekv_prefill_attn(const carekv_prefill_params* pp, const uint16_t* q, const uint16_t* k,
                                   const uint16_t* v, uint16_t* out, float* lse, void* stream) {
  CAREKV_REQUIRE(pp && q && k && v && out, "null argument");
  CAREKV_REQUIRE(pp->head_dim == 64 || pp->head_dim == 128, "head_dim must be 64 or 128");
  CAREKV_REQUIRE(pp->batch > 0 && pp->n_heads > 0 && pp->n_kv_heads > 0, "batch and head counts must be positive");
  CAREKV_REQUIRE(pp->n_heads % pp->n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
  CAREKV_REQUIRE(pp->seq_len > 0, "seq_len must be positive");
  // 32-bit buffer offsets reach one query block and one key tile past the end
  CAREKV_REQUIRE(((long)pp->seq_len + 128) * pp->head_dim * 2 < (1L << 31), "one head's sequence exceeds 2 GiB");
  PrefillArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = out; a.lse = lse;
  a.B = pp->batch; a.Hq = pp->n_heads; a.Hkv = pp->n_kv_heads; a.T = pp->seq_len; a.causal = pp->causal != 0;
  a.sm_log2 = pp->sm_scale * 1.4426950408889634f;
  const long nblk = (long)((pp->seq_len + 127) / 128) * pp->n_heads * pp->batch;
  CAREKV_REQUIRE(nblk < (1L << 31), "too many query blocks");
  const dim3 grid((unsigned)nblk);
  hipStream_t s = (hipStream_t)stream;
  if (pp->head_dim == 128) hipLaunchKernelGGL(prefill_attn_kernel<128>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(prefill_attn_kernel<64>, grid, dim3(256), 0, s, a);
  CAREKV_CHECK_LAUNCH("prefill_attn");
  return CAREKV_OK;
}

extern "C" int carekv_dequantize_rows(const int8_t* codes, const uint16_t* scale, int32_t rows, int32_t D,
                                      int32_t group, uint16_t* out, void* stream) {
  CAREKV_REQUIRE(codes && scale && out, "null argument");
  CAREKV_REQUIRE(group == 32 && D % 32 == 0 && D > 0, "kernels support group_size=32 and D % 32 == 0");
  if (rows <= 0) return CAREKV_OK;
  const long n = (long)rows * D;
  hipLaunchKernelGGL(dequantize_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     codes, scale, n, D, out);
  CAREKV_CHECK_LAUNCH("dequantize_rows");
  return CAREKV_OK;
}
