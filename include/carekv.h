/*
 * carekv.h -- C ABI of the MI355X-native CARE-KV quantized decode-attention
 * path (libcarekv_hip.so, HIP kernels built for gfx950).
 *
 * The reference (soeunida/CARE-KV-..., a PyTorch prototype) has no FFI; each
 * entry point below replaces the Python functions named in its comment
 * (paths relative to the reference root).  All functions return 0 on
 * success or a negative code; carekv_last_error() returns the message of the
 * last failure on the calling thread.  Every pointer is a device pointer
 * unless stated otherwise; work is enqueued on `stream` (a hipStream_t) and
 * nothing synchronises with the host.
 */
#ifndef CAREKV_H_
#define CAREKV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CAREKV_OK 0
#define CAREKV_EINVAL -1   /* bad shape / unsupported configuration      */
#define CAREKV_ELAUNCH -2  /* HIP launch or runtime error                */
#define CAREKV_ESPACE -3   /* workspace or slot arena too small          */

/* Paged cache of one layer, shared by all sequence slots.  Layout mirrors
 * CAREKVCache._init_buffers (cache.py:430-536) with the sequence slot as an
 * extra dimension next to the kv head:
 *   page index pg = (kv_head * n_seq + seq) * max_pages + page
 *   kcodes/vcodes  int8   [pg][page_size][row_bytes]   packed base codes,
 *                  or, with base_bits = 16, fp16 [pg][page_size][head_dim]:
 *                  the K_hat / V_hat side buffer of the KIVI-style base
 *                  (cache.py:487-499, base_K_hat_fp16); the scale and
 *                  master buffers are then unused and may be NULL
 *   kscale/vscale  int8   [pg][page_size][G]  (scale_mode 1: int8 codes)
 *                  fp16   [pg][page_size][G]  (scale_mode 0: raw fp16)
 *   kmaster/vmaster fp16  [pg]                 per-page master scale
 *   valid          int32  [pg]                 valid tokens per page
 *   has_meta       int8   [pg]                 PageMeta present (cache.py:530)
 *   k_slot         int32  [pg][D/kcg]          K residual slot id or -1
 *   v_slot         int32  [pg][page/vtb]       V residual slot id or -1
 *   k_err/v_err    fp16   [pg][..]             PageMeta.k/v_error_norm
 *   k_sketch       fp16   [pg][D/kcg][sketch]  PageMeta.k_sketch
 *   v_sq           fp32   [pg]                 sum of V_hat^2 over valid rows
 *   k_res/v_res    int8   [n_seq][n_slots][slot_bytes] residual slot arena
 *   k_res_scale/v_res_scale fp16 [n_seq][n_slots]
 *   next_slot      int32  [n_seq][2]           next free K / V slot id
 * Slot arenas are per sequence and shared by all layers of that sequence,
 * like the reference's per-sequence k_residual_buf (cache.py:522-527). */
typedef struct carekv_arena {
  int8_t* kcodes;
  int8_t* vcodes;
  void* kscale;
  void* vscale;
  uint16_t* kmaster;
  uint16_t* vmaster;
  int32_t* valid;
  int8_t* has_meta;
  int32_t* k_slot;
  int32_t* v_slot;
  uint16_t* k_err;
  uint16_t* v_err;
  uint16_t* k_sketch;
  float* v_sq;
  int8_t* k_res;
  uint16_t* k_res_scale;
  int8_t* v_res;
  uint16_t* v_res_scale;
  int32_t* next_slot;
  int32_t n_seq, n_kv_heads, max_pages, head_dim, base_bits, page_size, group_size;
  int32_t k_channel_group, v_token_block, sketch_dim, scale_mode, residual_bits, n_slots;
  int32_t hat_bits_k, hat_bits_v; /* base_bits = 16: the KIVI bits of a decode
                                   * append's K and V row (layer.py:197-202)  */
  /* Decode appends into int8-scale pages (scale_mode 1).  rescale_open = 0:
   * the reference's encoding, the row's scale codes against the page's fixed
   * master (cache.py:689-695; a page the decode opens keeps master 0 and its
   * rows read back as zero).  rescale_open = 1 (no reference counterpart):
   * the open page is re-encoded as write_base encodes its valid rows, from
   * their fp16 group scales in open_kscale / open_vscale, fp16
   * [n_kv_heads][n_seq][page_size][D/group] (the prompt writer fills the
   * rows of a partial last page, the append adds its row). */
  uint16_t* open_kscale;
  uint16_t* open_vscale;
  int32_t rescale_open;
  /* Packed KIVI-style base (no reference counterpart: the reference keeps the
   * KIVI K_hat / V_hat as fp16 side-buffer pages, cache.py:487-499, 800-865).
   * kivi_packed = 1 (base_bits 2, scale_mode 0, hat_bits_k = hat_bits_v = 2):
   * pages 0 .. n_packed[s]-1 of sequence s hold the prompt's full pages as
   * 2-bit codes, K against one per-channel scale vector per (kv head,
   * sequence) in kchan (fp16 [n_kv_heads][n_seq][head_dim], the scales of
   * quant_dequant_kivi_k over the prompt, kivi_helpers.py:35-47), V against
   * its row's per-token scale (quant_dequant_kivi_v, :50-59), kept in vscale
   * as fp16 [row][D/group] with every group of a row equal (kscale unused).
   * The later pages (the prompt's partial last page, the decode rows) are
   * the fp16 K_hat / V_hat rows of the side-buffer base in tail_k / tail_v,
   * [n_kv_heads][n_seq][tail_pages][page_size][head_dim]: page p of sequence
   * s at tail page p - n_packed[s].  kivi_packed = 0: all four unused. */
  int32_t kivi_packed;
  const uint16_t* kchan;
  const int32_t* n_packed;  /* device [n_seq] */
  uint16_t* tail_k;
  uint16_t* tail_v;
  int32_t tail_pages;
  /* Code-buffer page map of the views the library launches over; callers
   * set both to 0.  code_pages > 0: kcodes / vcodes / kscale / vscale hold
   * code_pages pages per (kv head, sequence) and page p of sequence s sits
   * at code page p - code_page_off[s]. */
  int32_t code_pages;
  const int32_t* code_page_off;
  /* streaming_store = 1 (no reference counterpart): the caller runs the
   * streaming fill store (carekv_store_pages with reuse_slots, and keep_base
   * on the packed bases) on every page a decode append fills, so
   * carekv_append_rows leaves such a page's metadata and slots to that store
   * instead of writing the reference's K_orig = K_hat metadata (no slots;
   * layer.py:1128-1146).  0: the reference's fill store in the append. */
  int32_t streaming_store;
} carekv_arena;

/* Store-time knobs, resolved on the host from CacheConfig and the
 * CAREKV_STORE_* environment (residual_store.py:104-114,379-422). */
typedef struct carekv_store_params {
  int32_t k_budget;        /* per-page K slots to keep (after mode/ratio/floor) */
  int32_t v_budget;        /* per-page V slots to keep                          */
  int32_t joint_budget;    /* joint store policy budget                         */
  int32_t joint;           /* 1: CAREKV_STORE_POLICY=joint                      */
  int32_t store_none;      /* 1: ratio budgets all <= 0 -> store nothing        */
  double sensitivity;      /* cfg.layer_sensitivity[layer]                      */
  int32_t sink_tokens;     /* prefill: is_sink = token_start < sink_tokens      */
  const float* sketch_proj;/* [k_channel_group][sketch_dim] fp32 (get_sketch_proj) */
  const uint16_t* k_hat;   /* base_bits = 16: fp16 K_hat / V_hat rows laid out  */
  const uint16_t* v_hat;   /* like K / V, written as the pages and the residual
                            * base (process_page with K_hat_override,
                            * residual_store.py:272-275); NULL otherwise       */
  int32_t keep_base;       /* 1: streaming store of pages the decode appends
                            * filled (packed bases): K / V are the pages' true
                            * rows, the pages keep their codes and scales and
                            * the residuals are taken against them as the decode
                            * reads them.  No reference counterpart: the
                            * reference stores such pages with K_orig = K_hat
                            * (layer.py:1128-1146), which leaves them no slots.
                            * 0: store as the prefill does                    */
  int32_t reuse_slots;     /* 1: the streaming fill store (no reference
                            * counterpart): a page's slot ids from an earlier
                            * store (a prompt's partial last page, metadata
                            * present) go, ascending, to its first selected
                            * candidates of their kind before new ids are
                            * taken; ids it no longer needs stay unused.
                            * A page without metadata holds none.  0: every
                            * selected candidate takes a new id             */
  /* process_page on a page carekv_write_base wrote (packed bases;
   * residual_store.py:239-464 with its K_codes / K_scale / V_codes / V_scale
   * arguments): int8 [n_jobs*page_size][head_dim] unpacked codes and fp16
   * [n_jobs*page_size][D/group] group scales the residuals are taken
   * against; the pages keep their base.  NULL: quantize K / V here.      */
  const int8_t* k_codes_in;
  const uint16_t* k_scale_in;
  const int8_t* v_codes_in;
  const uint16_t* v_scale_in;
  /* Packed KIVI arenas (kivi_packed = 1) take k_hat / v_hat for every job
   * (the residual base) and k_codes_in / v_codes_in / v_scale_in laid out as
   * there: a page below n_packed[seq] (set before the call) is written from
   * the 2-bit codes of carekv_kivi_codes, V with its row's per-token scale
   * in all D/group entries of the row (k_scale_in unused); a later page goes
   * to the fp16 tail as the side-buffer base writes it (its codes unused).
   * Slot ids follow job order across both kinds of page. */
} carekv_store_params;

/* One page write (prefill).  X rows for page j are X[j*page_size .. +page_size),
 * zero padded past num_valid (layer.py:254-271). */
typedef struct carekv_page_job {
  int32_t seq, kv_head, page, num_valid;
  int32_t token_start;     /* absolute position of the first row              */
  int32_t is_recent;       /* layer.py:275: p >= num_pages - 4                 */
} carekv_page_job;

/* Replaces CAREKVLayer._write_pages_for_kv_head's uniform branch
 * (layer.py:254-332): quantize + pack + int8 scales (quantizer.py:31-64,
 * 304-372; cache.py:592-654), then ResidualStoreManager.process_page
 * (residual_store.py:239-464) with deterministic slot ids (ascending in
 * job order, like the reference free-list pop(0), cache.py:548-560).
 * K, V: fp16 [n_jobs*page_size][head_dim].  Jobs are grouped by sequence:
 * group g is jobs [group_ptr[g], group_ptr[g+1]) (device int32 array), all of
 * one sequence and in the reference's call order (kv head major, page
 * minor).  workspace must hold carekv_store_workspace_bytes(arena, sp,
 * n_jobs) bytes.  Three launches: one pass over every page (codes, scales,
 * residual candidates, the store decision, the selected 4-bit payloads
 * staged in the workspace), the slot-id scan per group, the scatter of the
 * staged payloads to their slots. */
int carekv_store_pages(const carekv_arena* arena, const carekv_store_params* sp,
                       const uint16_t* K, const uint16_t* V, const carekv_page_job* jobs_dev,
                       int32_t n_jobs, const int32_t* group_ptr_dev, int32_t n_groups,
                       void* workspace, void* stream);
/* A prompt chunk of n_rows sequences, every kv head, as page jobs the
 * device generates (carekv_store_prefill): job j is (row b, kv head h,
 * page p) in row-major order over (n_rows, n_kv_heads, n_pages), n_pages =
 * ceil(n_tokens / page_size), with seq = rows[b], page = rows[n_rows +
 * b * n_kv_heads + h] + p, num_valid = min(page_size, n_tokens - p *
 * page_size), token_start = token_start + p * page_size, is_recent =
 * p >= n_pages - 4 (layer.py:254-275); one sequence group per row. */
typedef struct carekv_prefill_grid {
  int32_t n_rows;        /* B > 0                                            */
  int32_t n_tokens;      /* T > 0 tokens per row                             */
  int32_t token_start;   /* absolute position of the chunk's first token     */
  const int32_t* rows;   /* device int32 [n_rows + n_rows * n_kv_heads]      */
} carekv_prefill_grid;

/* carekv_store_pages over the jobs of a prompt chunk's grid, generated on
 * the device: what CAREKVLayer.prefill runs for every kv head
 * (_write_pages_for_kv_head, layer.py:204-334) in one call, without a host
 * job list.  K, V: fp16 [n_rows][n_kv_heads][n_pages * page_size]
 * [head_dim], zero padded past n_tokens; workspace as carekv_store_pages
 * with n_jobs = n_rows * n_kv_heads * n_pages. */
int carekv_store_prefill(const carekv_arena* arena, const carekv_store_params* sp,
                         const uint16_t* K, const uint16_t* V, const carekv_prefill_grid* grid,
                         void* workspace, void* stream);

/* Workspace bytes of a carekv_store_pages call with these arena, params and
 * job count (the staging area is sized by head_dim and the per-page
 * budgets); -1 on a null argument.  The int32 at workspace[4 * n_jobs] is
 * the call's status word: 0, or nonzero when a slot id would fall past
 * n_slots (those slots are dropped). */
int64_t carekv_store_workspace_bytes(const carekv_arena* arena, const carekv_store_params* sp, int32_t n_jobs);

/* One decode-token append per row (layer.py:1028-1146, cache.py:656-701):
 * quantize the row, pack it at (seq, kv_head, page, valid[pg]), encode its
 * scales against the page's fixed master (clamped at 1e-8) -- with
 * base_bits = 16, quant-dequant it alone in KIVI style (K per channel over
 * the one row, V per token, hat_bits_k/v; layer.py:1037-1075,
 * cache.py:820-838) and write the fp16 row --, bump valid, and
 * when the page becomes full write its PageMeta with the store run on
 * K_orig = K_hat (zero residual: no slots, zero errors and sketches).
 * dest_dev: int32 [n_rows][4] = (seq, kv_head, page, fresh); fresh=1 marks
 * a page just allocated by the caller (layer.py:1029-1035): it starts empty
 * with a zero master and no metadata, like the reference's zeroed buffers. */
int carekv_append_rows(const carekv_arena* arena, const uint16_t* k_rows, const uint16_t* v_rows,
                       const int32_t* dest_dev, int32_t n_rows, void* stream);

/* CAREKVCache.append_to_page (cache.py:656-701): rows already quantized by
 * the caller, int8 codes [n_rows][head_dim] and fp16 group scales
 * [n_rows][D/group], packed at (seq, kv_head, page, valid[pg]) with the
 * arena's scale encoding (as carekv_append_rows); dest_dev as there.  A page
 * the rows fill gets no metadata (the decode step's store on fill is not part
 * of the append).  Packed bases only. */
int carekv_append_coded_rows(const carekv_arena* arena, const int8_t* k_codes, const uint16_t* k_scale,
                             const int8_t* v_codes, const uint16_t* v_scale, const int32_t* dest_dev,
                             int32_t n_rows, void* stream);

/* Decode attention + comb+ex residual correction.  Replaces, per sequence
 * and kv head, CAREKVCache.read_base_concat (cache.py:720-772) + dequantize
 * (quantizer.py:67-82) + base attention (attention.py:1009-1022) +
 * vectorized_joint_correction (attention.py:576-957, KSCORE_LIVE=1 or the
 * KSCORE_LIVE=0 sketch proxy) over the kv head's query heads, output
 * half(O_base + dO) (attention.py:1036-1039). */
typedef struct carekv_decode_params {
  int32_t batch;           /* rows of q / out                                  */
  int32_t n_heads;         /* query heads; kv head = h / (n_heads/n_kv_heads)   */
  const int32_t* seq_slot; /* device [batch]: arena sequence slot of each row   */
  const int32_t* n_pages;  /* device [batch]: pages in use (page ids 0..n-1)    */
  int32_t max_pages_used;  /* host upper bound of n_pages[]                     */
  float sm_scale;          /* fp32(1/sqrt(head_dim))                            */
  float sensitivity;       /* cfg.layer_sensitivity[layer]                      */
  int32_t correction;      /* 0: base attention only                            */
  int32_t kind;            /* 0 both, 1 k, 2 v   (CAREKV_PREFILL_RESIDUAL_KIND) */
  int32_t joint;           /* 1 joint, 0 separate (route_policy)                */
  int32_t normalize;       /* CAREKV_SCORE_NORMALIZE                            */
  int32_t k_exact;         /* CAREKV_K_CORRECTION_MODE: 1 exact, 0 linear       */
  float k_corr_scale;      /* CAREKV_K_CORRECTION_SCALE (linear mode)           */
  float lambda_k, lambda_v;/* CAREKV_KSCORE_LAMBDA_K/V                          */
  int32_t budget_ratio;    /* 0 absolute (abs_k/abs_v), 1 ratio (ratio_k/v)     */
  int32_t abs_k, abs_v;    /* _resolve_read_budgets, multiplier applied         */
  double ratio_k, ratio_v;
  int32_t k_cap, v_cap;    /* max stored K / V slots per page                   */
  int32_t split_pages;     /* pages per work-group in the streaming pass        */
  void* phase_events;      /* optional timing hook: NULL, or a host array of 5
                            * hipEvent_t made by the caller, recorded on
                            * `stream` before the streaming kernel and after the
                            * streaming, select, apply and combine kernels (no
                            * reference counterpart; with correction off the
                            * last two are recorded right after select)       */
  int32_t k_proxy;         /* 0: the query-aware K score (CAREKV_KSCORE_LIVE=1,
                            * attention.py:704-717); 1: the sketch proxy
                            * mass * |q_sketch . k_sketch| * boundary * vdiff
                            * * sens (KSCORE_LIVE=0, attention.py:718-725, the
                            * score of ResidualRouter.route,
                            * residual_router.py:160-198)                     */
  const float* sketch_proj;/* device [k_channel_group][sketch_dim] fp32, the
                            * get_sketch_proj matrix (residual_store.py:206-214);
                            * required when k_proxy = 1                       */
  int32_t route_policy;    /* 0: `joint` decides (joint / separate); 2 k_first,
                            * 3 adaptive: the policies of ResidualRouter.route
                            * (residual_router.py:322-365)                     */
  int32_t adaptive_score;  /* read_budget_mode adaptive_score: per-kind score
                            * thresholds after the policy (:366-410)          */
  double rel_threshold, abs_threshold; /* CAREKV_READ_RELATIVE/ABSOLUTE_THRESHOLD */
  int32_t min_keep;        /* CAREKV_READ_MIN_KEEP                             */
  unsigned long long* read_counts; /* optional device [3], NULL to skip: the
                            * call adds the K slots and V blocks it selected
                            * and the queries it corrected (the debug stats
                            * k_slots_read / v_slots_read / n_queries,
                            * attention.py:358-372,944-946)                   */
  int32_t packed_pages_used; /* kivi_packed arenas: host upper bounds over the */
  int32_t tail_pages_used;   /* rows of min(n_pages, n_packed) and of
                              * n_pages - n_packed (ignored otherwise)         */
} carekv_decode_params;

/* q, out: fp16 [batch][n_heads][head_dim].  The first int32 of the
 * workspace is the call's status word: 0, or nonzero when a page holds more
 * stored residual slots than k_cap / v_cap (those slots are left out of the
 * scoring); it is written on the device, read it after the stream is done.
 * diag (optional, NULL to skip):
 * int32 [batch][n_heads][diag_cap] selected candidates, each encoded
 * kind<<30 | page<<3 | sub (kind 0 = K with sub = channel group,
 * 1 = V with sub = token block), sorted ascending, -1 padded. */
int carekv_decode_attn(const carekv_arena* arena, const carekv_decode_params* dp, const uint16_t* q,
                       uint16_t* out, void* workspace, int64_t workspace_bytes, int32_t* diag,
                       int32_t diag_cap, void* stream);
int64_t carekv_decode_workspace_bytes(const carekv_arena* arena, const carekv_decode_params* dp);

/* No reference counterpart: carekv_decode_attn for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as carekv_decode_attn
 * without the workspace: the step's workspace is a file-scope device array
 * of CAREKV_STATIC_SCRATCH_BYTES per GPU, held by each GPU the library runs
 * on until the process ends.  Steps needing more workspace than that
 * (carekv_decode_workspace_bytes) fail with CAREKV_ESPACE and a message.
 * The call allocates nothing; the stream's device must be current.  Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two threads) race.  The overflow status word lives in the
 * array and is not read back; check a configuration with carekv_decode_attn
 * first. */
#define CAREKV_STATIC_SCRATCH_BYTES (64L << 20)
int carekv_decode_attn_static(const carekv_arena* arena, const carekv_decode_params* dp, const uint16_t* q,
                              uint16_t* out, int32_t* diag, int32_t diag_cap, void* stream);

/* read_base_concat (cache.py:720-772) for one (seq, kv_head): unpacked int8
 * codes [N][D] and fp16 scales [N][G] of the valid rows of the listed pages
 * (int8 scales expanded as half(code * master)).  page_ids_dev: int32
 * [n_pages] page ids, or NULL for pages 0..n_pages-1; row_start_dev: int32
 * [n_pages] exclusive prefix of the listed pages' valid counts (host
 * computed). */
int carekv_read_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                      const int32_t* page_ids_dev, const int32_t* row_start_dev, int8_t* kc, uint16_t* ks,
                      int8_t* vc, uint16_t* vs, void* stream);

/* CAREKVCache.write_base (cache.py:617-654) of one page: k_codes / v_codes
 * int8 [page_size][head_dim] unpacked codes, k_scale / v_scale fp16
 * [page_size][D/group]; packs the codes, encodes the scales (int8 codes
 * under the page's fp16 master, cache.py:592-604, or fp16) and sets the
 * page's valid count. */
int carekv_write_base(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t page, const int8_t* k_codes,
                      const uint16_t* k_scale, const int8_t* v_codes, const uint16_t* v_scale, int32_t num_valid,
                      void* stream);

/* pack_codes_2d / unpack_codes_2d (quantizer.py:257-383): int8 codes
 * [rows][D] <-> packed [rows][D*bits/8]; INT3 packs 8 codes into a 24-bit
 * little-endian word, INT2 4 and INT4 2 codes into a byte, LSB first.  The
 * 1-D pack_int* / unpack_int* (quantizer.py:147-249) are one row of the
 * zero-padded codes.  D a multiple of 8 (INT3), 4 (INT2) or 2 (INT4). */
int carekv_pack_codes(const int8_t* codes, int64_t rows, int32_t D, int32_t bits, int8_t* packed, void* stream);
int carekv_unpack_codes(const int8_t* packed, int64_t rows, int32_t D, int32_t bits, int8_t* codes, void* stream);

/* pack_4bit / unpack_4bit (residual_store.py:121-146): x float32 (x_fp16 = 0)
 * or fp16, numel values -> packed int8 [(numel + 1) / 2], scale fp16 [1]
 * (s = max|x| / 7 in the input's arithmetic); unpack gives float32
 * code * float(scale). */
int carekv_pack_4bit(const void* x, int32_t x_fp16, int64_t numel, int8_t* packed, uint16_t* scale, void* stream);
int carekv_unpack_4bit(const int8_t* packed, const uint16_t* scale, int64_t numel, float* out, void* stream);

/* quantize / dequantize (quantizer.py:31-82) on float32 rows, in fp32
 * arithmetic: codes int8 [rows][D], scale float32 [rows][D/group]; group 32. */
int carekv_quantize_rows_f32(const float* x, int64_t rows, int32_t D, int32_t bits, int32_t group, int8_t* codes,
                             float* scale, void* stream);
int carekv_dequantize_rows_f32(const int8_t* codes, const float* scale, int64_t rows, int32_t D, int32_t group,
                               float* out, void* stream);

/* Symmetric per-group quantizer on fp16 rows (quantizer.py:31-64, fp16
 * arithmetic) with optional bit packing (quantizer.py:364-372).
 * x fp16 [rows][D]; codes int8 [rows][D] (or packed [rows][row_bytes] when
 * pack != 0); scale fp16 [rows][D/group]. */
int carekv_quantize_rows(const uint16_t* x, int32_t rows, int32_t D, int32_t bits, int32_t group,
                         int32_t pack, int8_t* codes, uint16_t* scale, void* stream);

/* KIVI-style quant-dequant (kivi_helpers.py:35-59), in fp16 arithmetic:
 * x, out fp16 [n_mat][rows][D].  per_channel != 0: quant_dequant_kivi_k,
 * one scale per (matrix, column) over the rows (K over the sequence);
 * per_channel == 0: quant_dequant_kivi_v, one scale per row (V per token).
 * scale = half(max|x| / qmax), code = clamp(rint(half(x / scale))),
 * out = half(code * scale); an all-zero channel (or a zero component of a
 * single-row K) gives NaN, as in the reference.  bits 2, 3 or 4; D <= 1024. */
int carekv_kivi_qdq(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits, int32_t per_channel,
                    uint16_t* out, void* stream);

/* No reference counterpart (the reference keeps only the fp16 K_hat / V_hat
 * of carekv_kivi_qdq): the codes and scales behind them, for the packed KIVI
 * pages.  codes int8 [n_mat][rows][D], code = clamp(rint(half(x / scale)))
 * and 0 where that is NaN; scale fp16 [n_mat][D] (per_channel) or
 * [n_mat][rows], NaN where max|x| = 0 (so that half(code * scale) is
 * carekv_kivi_qdq's NaN there).  half(code * scale) equals carekv_kivi_qdq
 * bit for bit up to the sign of zero, except where a nonzero max|x| gives a
 * scale of 0 in fp16 (max|x| < 2^-25 qmax): there the exact zeros of x
 * dequantise to 0 instead of NaN. */
int carekv_kivi_codes(const uint16_t* x, int32_t n_mat, int32_t rows, int32_t D, int32_t bits, int32_t per_channel,
                      int8_t* codes, uint16_t* scale, void* stream);

/* read_base_hat_concat of the side-buffer base (cache.py:487-499, 800-865)
 * for base_bits = 16 and packed KIVI arenas: the fp16 K_hat / V_hat rows of
 * pages page_ids_dev[0..n_pages) (or 0..n_pages-1 when NULL) of (seq,
 * kv_head), page p's valid rows at k_hat / v_hat rows row_start_dev[p]..
 * (fp16 [rows][head_dim]); a packed page dequantises half(code * scale). */
int carekv_read_hat_pages(const carekv_arena* arena, int32_t seq, int32_t kv_head, int32_t n_pages,
                          const int32_t* page_ids_dev, const int32_t* row_start_dev, uint16_t* k_hat,
                          uint16_t* v_hat, void* stream);

/* Prefill attention over dequantised K/V: CAREKVLayer._causal_attention_pure
 * (layer.py:935-972) for a batch of sequences, with GQA heads read in place
 * instead of repeat_interleave'd (layer.py:774-775).  q fp16
 * [batch][n_heads][seq_len][head_dim], k/v fp16 [batch][n_kv_heads][seq_len]
 * [head_dim] (post-RoPE K_hat, V_hat), out fp16 like q.  Scores are the fp32
 * product times sm_scale; causal != 0 masks tokens after the query (the
 * attention_mask=None branch, layer.py:958-962).  The (T, T) weights are not
 * materialised: lse (optional, fp32 [batch][n_heads][seq_len]) receives the
 * natural log-sum-exp of each query's scaled scores, so that any weight is
 * exp(score * sm_scale - lse).  head_dim 64 or 128. */
typedef struct carekv_prefill_params {
  int32_t batch, n_heads, n_kv_heads, seq_len, head_dim, causal;
  float sm_scale;
} carekv_prefill_params;

int carekv_prefill_attn(const carekv_prefill_params* params, const uint16_t* q, const uint16_t* k,
                        const uint16_t* v, uint16_t* out, float* lse, void* stream);

/* Prefill in carekv_eval mode: CAREKVLayer._apply_sparse_prefill_correction_eval
 * (layer.py:363-456) over the causal base attention, as prefill calls it
 * (layer.py:792-806).  For every query head h and row t, over the row's
 * tokens j <= t with a_j the fp16 base weight (the row's softmax of
 * q.K_hat_j / sqrt(D) in fp32, cast to fp16; layer.py:963), r_k =
 * half(K - K_hat), r_v = half(V - V_hat):
 *   v_score = a ||r_v|| ||V_hat_j - o|| (v_score_norm: a ||r_v||),
 *   k_score = a |q.r_k / sqrt(D)| ||V_hat_j - o||,
 *   score by kind (both: v + k, or v / mean|v| + k / mean|k| when normalize),
 *   the top min(max(min_residuals, int((t + 1) ratio)), t + 1) tokens (ties
 *   to the lower index), and
 *   out = half(o + sum a r_v + k_corr_scale sum a clamp(q.r_k / sqrt(D),
 *   -2, 2) (V_hat_j - o)).
 * q, o_base, out fp16 [batch][n_heads][seq_len][head_dim] (o_base the base
 * output of carekv_prefill_attn over K_hat / V_hat); k, v (true post-RoPE
 * rows), k_hat, v_hat fp16
 * [batch][n_kv_heads][seq_len][head_dim].  diag (optional, diag_cap > 0):
 * int32 [batch][n_heads][seq_len][diag_cap] the selected token indices,
 * ascending, -1 padded.  seq_len <= 8192, head_dim 64 or 128. */
typedef struct carekv_prefill_eval_params {
  int32_t batch, n_heads, n_kv_heads, seq_len, head_dim;
  double ratio;           /* CAREKV_PREFILL_RESIDUAL_RATIO (default cfg.read_budget_ratio) */
  int32_t min_residuals;  /* CAREKV_PREFILL_MIN_RESIDUALS                     */
  int32_t kind;           /* CAREKV_PREFILL_RESIDUAL_KIND: 0 both, 1 k, 2 v   */
  int32_t v_score_norm;   /* CAREKV_V_SCORE: 1 norm, 0 output_aware           */
  int32_t normalize;      /* CAREKV_SCORE_NORMALIZE                           */
  float k_corr_scale;     /* CAREKV_K_CORRECTION_SCALE                        */
  int32_t diag_cap;
} carekv_prefill_eval_params;

int carekv_prefill_eval(const carekv_prefill_eval_params* params, const uint16_t* q, const uint16_t* k,
                        const uint16_t* v, const uint16_t* k_hat, const uint16_t* v_hat, const uint16_t* o_base,
                        uint16_t* out, int32_t* diag, void* stream);

/* Prefill-time sparse correction of CAREKVLayer.prefill in carekv_stored
 * mode (layer.py:780-838) with the vectorized correction over all
 * kv_group x T queries of each kv head (layer.py:538-557): for every prompt
 * row t in [row_begin, row_begin + n_rows) and query head h,
 *   out[t - row_begin][h] = half(O_base + vectorized_joint_correction(...))
 * with the base attention of _causal_attention_pure (fp32 scores, softmax
 * weights cast to fp16, layer.py:952-965) over the prompt's first t + 1
 * tokens, scored against the stored slots of every page of the prompt (the
 * candidates of pages after row t score 0 but count towards the
 * normalisation and the budgets, as in the reference).
 * The arena's sequence `seq` must hold exactly the prompt's pages
 * (carekv_store_pages over tokens 0..n_tokens-1).  k_hat / v_hat are the
 * page writer's dequantised prompt (layer.py:331-334: half(code * fp16 group
 * scale), before the int8 requantisation of the page scales; the KIVI
 * quant-dequant for the side-buffer bases), fp16 [n_kv_heads][n_tokens]
 * [head_dim]; lse is carekv_prefill_attn's natural log-sum-exp of the same
 * rows, fp32 [n_heads][n_tokens]. */
typedef struct carekv_prefill_corr_params {
  int32_t seq;        /* arena sequence slot holding the prompt              */
  int32_t n_tokens;   /* prompt length T                                     */
  int32_t row_begin;  /* first prompt row to correct                         */
  int32_t n_rows;     /* rows to correct                                     */
  const uint16_t* k_hat;
  const uint16_t* v_hat;
  const float* lse;
} carekv_prefill_corr_params;

/* read: the read knobs, as for a decode step; its batch, seq_slot, n_pages
 * and max_pages_used are ignored, correction must be 1 and k_proxy 0.
 * q, out: fp16 [n_rows][n_heads][head_dim] (the prompt rows' post-RoPE
 * queries, row-major over the rows).  diag as carekv_decode_attn, per row. */
int carekv_prefill_correct(const carekv_arena* arena, const carekv_decode_params* read,
                           const carekv_prefill_corr_params* rows, const uint16_t* q, uint16_t* out,
                           void* workspace, int64_t workspace_bytes, int32_t* diag, int32_t diag_cap,
                           void* stream);
int64_t carekv_prefill_correct_workspace_bytes(const carekv_arena* arena, const carekv_decode_params* read,
                                               const carekv_prefill_corr_params* rows);

/* dequantize (quantizer.py:67-82): out fp16 [rows][D] = half(code * scale)
 * from unpacked int8 codes [rows][D] and fp16 group scales [rows][D/group]
 * as carekv_quantize_rows (pack = 0) writes them; group must be 32. */
int carekv_dequantize_rows(const int8_t* codes, const uint16_t* scale, int32_t rows, int32_t D, int32_t group,
                           uint16_t* out, void* stream);

const char* carekv_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* CAREKV_H_ */
