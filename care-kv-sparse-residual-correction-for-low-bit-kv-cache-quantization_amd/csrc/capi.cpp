// C ABI plumbing shared by all entry points: per-thread error string and
// arena validation.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "host_util.h"

namespace carekv {

static thread_local char g_err[512] = "";

char* last_error_buf() { return g_err; }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

bool check_arena(const carekv_arena& A) {
  const bool hat = A.base_bits == 16;
  if (!A.kcodes || !A.vcodes || (!hat && (!A.kscale || !A.vscale)) || !A.valid || !A.has_meta || !A.k_slot ||
      !A.v_slot ||
      !A.k_err || !A.v_err || !A.k_sketch || !A.v_sq || !A.k_res || !A.k_res_scale || !A.v_res ||
      !A.v_res_scale || !A.next_slot) {
    set_error("arena has a null buffer");
    return false;
  }
  if (!hat && A.scale_mode == 1 && (!A.kmaster || !A.vmaster)) {
    set_error("scale_mode=int8 needs master buffers");
    return false;
  }
  if (!hat && A.scale_mode == 1 && A.rescale_open && (!A.open_kscale || !A.open_vscale)) {
    set_error("rescale_open needs the open pages' fp16 scales (open_kscale, open_vscale)");
    return false;
  }
  if (A.page_size != 16 || A.group_size != 32 || A.k_channel_group != 32 || A.v_token_block != 4) {
    set_error("kernels support page_size=16, group_size=32, k_channel_group=32, v_token_block=4 "
              "(got %d/%d/%d/%d)", A.page_size, A.group_size, A.k_channel_group, A.v_token_block);
    return false;
  }
  if (A.head_dim != 64 && A.head_dim != 128) {
    set_error("kernels support head_dim 64 or 128 (got %d)", A.head_dim);
    return false;
  }
  if ((A.base_bits < 2 || A.base_bits > 4) && !hat) {
    set_error("base_bits must be 2, 3, 4 or 16 (fp16 side buffer) (got %d)", A.base_bits);
    return false;
  }
  if (hat && (A.hat_bits_k < 2 || A.hat_bits_k > 4 || A.hat_bits_v < 2 || A.hat_bits_v > 4)) {
    set_error("base_bits=16 needs hat_bits_k/v in 2..4 (got %d/%d)", A.hat_bits_k, A.hat_bits_v);
    return false;
  }
  if (A.scale_mode != 0 && A.scale_mode != 1) {
    set_error("scale_mode must be 0 (fp16) or 1 (int8)");
    return false;
  }
  if (A.code_pages != 0 || A.code_page_off) {
    set_error("code_pages / code_page_off are set by the library on its own views (callers pass 0)");
    return false;
  }
  if (A.kivi_packed &&
      (A.base_bits != 2 || A.scale_mode != 0 || A.hat_bits_k != 2 || A.hat_bits_v != 2 || !A.kchan ||
       !A.n_packed || !A.tail_k || !A.tail_v || A.tail_pages <= 0)) {
    set_error("a packed KIVI arena needs base_bits 2, scale_mode 0 (fp16), hat_bits_k = hat_bits_v = 2, kchan, "
              "n_packed, tail_k, tail_v and tail_pages > 0");
    return false;
  }
  if (A.sketch_dim <= 0 || A.sketch_dim > 64) {
    set_error("sketch_dim must be in 1..64 (got %d)", A.sketch_dim);
    return false;
  }
  if (A.n_seq <= 0 || A.n_kv_heads <= 0 || A.max_pages <= 0 || A.n_slots <= 0) {
    set_error("arena dimensions must be positive");
    return false;
  }
  // the kernels address one (kv head, sequence) row of pages and one
  // sequence's slot arena with 32-bit buffer offsets below 2^31
  const long row_span = (long)A.max_pages * kPage * row_bytes(A.head_dim, A.base_bits);
  const long slot_span = (long)A.n_slots * (kPage * 32 / 2 > kVtb * A.head_dim / 2 ? kPage * 32 / 2 : kVtb * A.head_dim / 2);
  if (row_span >= (1L << 31) || slot_span >= (1L << 31)) {
    set_error("a row of pages or a sequence's slot arena exceeds 2 GiB");
    return false;
  }
  return true;
}

}  // namespace carekv

extern "C" const char* carekv_last_error(void) { return carekv::g_err; }
