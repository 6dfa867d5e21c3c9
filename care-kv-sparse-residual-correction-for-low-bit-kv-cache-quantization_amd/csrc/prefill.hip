// Prefill attention over dequantised K/V (CAREKVLayer._causal_attention_pure,
// layer.py:935-972) on v_mfma_f32_16x16x32_f16, flash style: the (T, T)
// score and weight matrices are never materialised; the kernel returns O and,
// optionally, the per-row log-sum-exp from which any weight can be rebuilt.
//
// One work-group per (block of 128 queries, query head, sequence), 4 waves of
// 32 queries.  K and V tiles of 64 tokens are staged in LDS (double
// buffered, one barrier per tile; the next tile's global loads are in flight
// while the current one is used):
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
// bytes, which keeps both LDS read patterns free of bank conflicts.
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
__global__ __launch_bounds__(256, 2) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int KT = 64;              // tokens per K/V tile
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

  const int qblk = gridDim.x - 1 - blockIdx.x;  // the longest (latest) blocks start first
  const int h = blockIdx.y, b = blockIdx.z;
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
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(c < KT * CHR ? rk : rv, off, 0, 0);
      stg[k][0] = v[0]; stg[k][1] = v[1]; stg[k][2] = v[2]; stg[k][3] = v[3];
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = threadIdx.x + 256 * k;
      const int rc = c % (KT * CHR), row = rc / CHR, col = rc % CHR;
      char* dst = lds + buf * BUF + (c < KT * CHR ? row * KRS : KBUF + row * VRS) + col * 16;
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
      // ---- S^T = K_hat Q^T
      float4_t s[4][2];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
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
      // ---- scale, mask (the wave's diagonal and the end of the sequence)
      const bool edge = (a.causal && t0 + KT - 1 > qw0) || t0 + KT > T;
      float p[4][2][4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int qi = qw0 + 16 * qb + c16;
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float x = s[tt][qb][i] * a.sm_log2;
            if (edge) {
              const int tok = t0 + 16 * tt + 4 * g + i;
              if (tok >= T || (a.causal && tok > qi)) x = -INFINITY;
            }
            p[tt][qb][i] = x;
            mx = fmaxf(mx, x);
          }
        mx = pair32_max(pair16_max(mx));
        const float m_new = fmaxf(m_run[qb], mx);  // finite: token 0 is visible to every query
        const float f = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
        m_run[qb] = m_new;
        float ls = 0.f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = __builtin_amdgcn_exp2f(p[tt][qb][i] - m_new);
            p[tt][qb][i] = e;
            ls += e;
          }
        l_run[qb] = l_run[qb] * f + ls;  // this lane's tokens; summed over the lane groups at the end
        if (__builtin_expect(__any(f != 1.f), 0)) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[qb][dt] *= f;
        }
      }
      // ---- O^T += V_hat^T P^T, 32 tokens per step
#pragma unroll
      for (int u = 0; u < 2; ++u) {
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

}  // namespace carekv

using namespace carekv;

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
  const dim3 grid((pp->seq_len + 127) / 128, pp->n_heads, pp->batch);
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
