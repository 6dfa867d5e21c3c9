// Host-side helpers for the C ABI: error reporting and template dispatch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdio.h>

#include <type_traits>

#include "carekv.h"

namespace carekv {

char* last_error_buf();
void set_error(const char* fmt, ...);

#define CAREKV_REQUIRE(cond, msg)                                        \
  do {                                                                   \
    if (!(cond)) {                                                       \
      if ((const char*)(msg) != carekv::last_error_buf())                \
        carekv::set_error("%s: %s", __func__, (const char*)(msg));       \
      return CAREKV_EINVAL;                                              \
    }                                                                    \
  } while (0)

#define CAREKV_CHECK_LAUNCH(what)                                                           \
  do {                                                                                      \
    hipError_t e_ = hipGetLastError();                                                      \
    if (e_ != hipSuccess) {                                                                 \
      carekv::set_error("%s: launch of %s failed: %s", __func__, what, hipGetErrorString(e_)); \
      return CAREKV_ELAUNCH;                                                                \
    }                                                                                       \
  } while (0)

// Validate the arena against what the kernels support.  On failure the
// message is left in last_error_buf().
bool check_arena(const carekv_arena& A);

template <typename F>
int dispatch_db(int D, int bits, F&& f) {
  using I64 = std::integral_constant<int, 64>;
  using I128 = std::integral_constant<int, 128>;
  using B2 = std::integral_constant<int, 2>;
  using B3 = std::integral_constant<int, 3>;
  using B4 = std::integral_constant<int, 4>;
  if (D == 64) {
    if (bits == 2) return f(I64{}, B2{});
    if (bits == 3) return f(I64{}, B3{});
    if (bits == 4) return f(I64{}, B4{});
  } else if (D == 128) {
    if (bits == 2) return f(I128{}, B2{});
    if (bits == 3) return f(I128{}, B3{});
    if (bits == 4) return f(I128{}, B4{});
  }
  set_error("unsupported head_dim=%d / base_bits=%d (kernels: head_dim 64|128, bits 2|3|4)", D, bits);
  return CAREKV_EINVAL;
}

// dispatch_db plus the scale encoding (0: fp16 scales, 1: int8 codes).
template <typename F>
int dispatch_dbs(int D, int bits, int scale_mode, F&& f) {
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  return dispatch_db(D, bits, [&](auto d, auto bb) {
    if (scale_mode == 1) return f(d, bb, S1{});
    return f(d, bb, S0{});
  });
}

// dispatch_dbs plus base_bits = 16 (the fp16 side buffer; scale mode 0):
// for the kernels that implement that base.
template <typename F>
int dispatch_dbs16(int D, int bits, int scale_mode, F&& f) {
  using B16 = std::integral_constant<int, 16>;
  using S0 = std::integral_constant<int, 0>;
  if (bits == 16) {
    if (D == 64) return f(std::integral_constant<int, 64>{}, B16{}, S0{});
    if (D == 128) return f(std::integral_constant<int, 128>{}, B16{}, S0{});
    set_error("unsupported head_dim=%d for the fp16 base (64|128)", D);
    return CAREKV_EINVAL;
  }
  return dispatch_dbs(D, bits, scale_mode, f);
}

}  // namespace carekv
