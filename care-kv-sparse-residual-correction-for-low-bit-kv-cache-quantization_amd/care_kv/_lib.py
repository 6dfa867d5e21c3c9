"""ctypes binding of libcarekv_hip.so (C ABI declared in include/carekv.h).

The library is required: every entry point raises if it is missing or if
the tensors handed to it are not on a HIP device.  There is no fallback.
"""
from __future__ import annotations

import collections
import ctypes as C
import os
import threading
import warnings

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcarekv_hip.so")
_lib = None
_lock = threading.Lock()


class CarekvError(RuntimeError):
    pass


class Arena(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "kcodes", "vcodes", "kscale", "vscale", "kmaster", "vmaster", "valid", "has_meta", "k_slot", "v_slot",
        "k_err", "v_err", "k_sketch", "v_sq", "k_res", "k_res_scale", "v_res", "v_res_scale", "next_slot")] + \
        [(n, C.c_int32) for n in (
            "n_seq", "n_kv_heads", "max_pages", "head_dim", "base_bits", "page_size", "group_size",
            "k_channel_group", "v_token_block", "sketch_dim", "scale_mode", "residual_bits", "n_slots",
            "hat_bits_k", "hat_bits_v")] + \
        [("open_kscale", C.c_void_p), ("open_vscale", C.c_void_p), ("rescale_open", C.c_int32)] + \
        [("kivi_packed", C.c_int32), ("kchan", C.c_void_p), ("n_packed", C.c_void_p), ("tail_k", C.c_void_p),
         ("tail_v", C.c_void_p), ("tail_pages", C.c_int32), ("code_pages", C.c_int32),
         ("code_page_off", C.c_void_p), ("streaming_store", C.c_int32)]


class StoreParams(C.Structure):
    _fields_ = [("k_budget", C.c_int32), ("v_budget", C.c_int32), ("joint_budget", C.c_int32),
                ("joint", C.c_int32), ("store_none", C.c_int32), ("sensitivity", C.c_double),
                ("sink_tokens", C.c_int32), ("sketch_proj", C.c_void_p), ("k_hat", C.c_void_p),
                ("v_hat", C.c_void_p), ("keep_base", C.c_int32), ("reuse_slots", C.c_int32), ("k_codes_in", C.c_void_p),
                ("k_scale_in", C.c_void_p), ("v_codes_in", C.c_void_p), ("v_scale_in", C.c_void_p)]


class PrefillGrid(C.Structure):
    _fields_ = [("n_rows", C.c_int32), ("n_tokens", C.c_int32), ("token_start", C.c_int32), ("rows", C.c_void_p)]


class DecodeParams(C.Structure):
    _fields_ = [("batch", C.c_int32), ("n_heads", C.c_int32), ("seq_slot", C.c_void_p), ("n_pages", C.c_void_p),
                ("max_pages_used", C.c_int32), ("sm_scale", C.c_float), ("sensitivity", C.c_float),
                ("correction", C.c_int32), ("kind", C.c_int32), ("joint", C.c_int32), ("normalize", C.c_int32),
                ("k_exact", C.c_int32), ("k_corr_scale", C.c_float), ("lambda_k", C.c_float),
                ("lambda_v", C.c_float), ("budget_ratio", C.c_int32), ("abs_k", C.c_int32), ("abs_v", C.c_int32),
                ("ratio_k", C.c_double), ("ratio_v", C.c_double), ("k_cap", C.c_int32), ("v_cap", C.c_int32),
                ("split_pages", C.c_int32), ("phase_events", C.c_void_p), ("k_proxy", C.c_int32),
                ("sketch_proj", C.c_void_p), ("route_policy", C.c_int32), ("adaptive_score", C.c_int32),
                ("rel_threshold", C.c_double), ("abs_threshold", C.c_double), ("min_keep", C.c_int32),
                ("read_counts", C.c_void_p), ("packed_pages_used", C.c_int32), ("tail_pages_used", C.c_int32)]


class PrefillParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("batch", "n_heads", "n_kv_heads", "seq_len", "head_dim", "causal")] + \
        [("sm_scale", C.c_float)]


class PrefillCorrParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("seq", "n_tokens", "row_begin", "n_rows")] + \
        [(n, C.c_void_p) for n in ("k_hat", "v_hat", "lse")]


class PrefillEvalParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("batch", "n_heads", "n_kv_heads", "seq_len", "head_dim")] + \
        [("ratio", C.c_double)] + [(n, C.c_int32) for n in ("min_residuals", "kind", "v_score_norm", "normalize")] + \
        [("k_corr_scale", C.c_float), ("diag_cap", C.c_int32)]


# page job: int32 x 6 (seq, kv_head, page, num_valid, token_start, is_recent)
PAGE_JOB_INTS = 6

EXPORTS = ["carekv_store_pages", "carekv_store_prefill", "carekv_store_workspace_bytes", "carekv_append_rows", "carekv_decode_attn",
           "carekv_decode_workspace_bytes", "carekv_read_pages", "carekv_quantize_rows", "carekv_prefill_attn",
           "carekv_dequantize_rows", "carekv_kivi_qdq", "carekv_prefill_correct",
           "carekv_prefill_correct_workspace_bytes", "carekv_decode_attn_static", "carekv_write_base", "carekv_append_coded_rows",
           "carekv_pack_codes", "carekv_unpack_codes", "carekv_pack_4bit", "carekv_unpack_4bit",
           "carekv_quantize_rows_f32", "carekv_dequantize_rows_f32", "carekv_kivi_codes", "carekv_read_hat_pages",
           "carekv_prefill_eval", "carekv_last_error"]

# bytes of the per-GPU static workspace of carekv_decode_attn_static
# (CAREKV_STATIC_SCRATCH_BYTES in include/carekv.h)
STATIC_SCRATCH_BYTES = 64 << 20


def lib_path() -> str:
    return _LIB_PATH


def load(path: str | None = None):
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = path or os.environ.get("CAREKV_LIB") or _LIB_PATH
        if not os.path.exists(p):
            raise CarekvError(f"{p} not found: build it with `python -m care_kv.build` "
                              "(or __graft_entry__.build()); there is no non-HIP fallback")
        lib = C.CDLL(p)
        vp, i32, i64 = C.c_void_p, C.c_int32, C.c_int64
        lib.carekv_last_error.restype = C.c_char_p
        lib.carekv_store_workspace_bytes.restype = i64
        lib.carekv_store_workspace_bytes.argtypes = [C.POINTER(Arena), C.POINTER(StoreParams), i32]
        lib.carekv_store_pages.restype = C.c_int
        lib.carekv_store_pages.argtypes = [C.POINTER(Arena), C.POINTER(StoreParams), vp, vp, vp, i32, vp, i32, vp, vp]
        lib.carekv_store_prefill.restype = C.c_int
        lib.carekv_store_prefill.argtypes = [C.POINTER(Arena), C.POINTER(StoreParams), vp, vp, C.POINTER(PrefillGrid),
                                             vp, vp]
        lib.carekv_append_rows.restype = C.c_int
        lib.carekv_append_rows.argtypes = [C.POINTER(Arena), vp, vp, vp, i32, vp]
        lib.carekv_decode_workspace_bytes.restype = i64
        lib.carekv_decode_workspace_bytes.argtypes = [C.POINTER(Arena), C.POINTER(DecodeParams)]
        lib.carekv_decode_attn.restype = C.c_int
        lib.carekv_decode_attn.argtypes = [C.POINTER(Arena), C.POINTER(DecodeParams), vp, vp, vp, i64, vp, i32, vp]
        lib.carekv_decode_attn_static.restype = C.c_int
        lib.carekv_decode_attn_static.argtypes = [C.POINTER(Arena), C.POINTER(DecodeParams), vp, vp, vp, i32, vp]
        lib.carekv_read_pages.restype = C.c_int
        lib.carekv_read_pages.argtypes = [C.POINTER(Arena), i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]
        lib.carekv_append_coded_rows.restype = C.c_int
        lib.carekv_append_coded_rows.argtypes = [C.POINTER(Arena), vp, vp, vp, vp, vp, i32, vp]
        lib.carekv_quantize_rows.restype = C.c_int
        lib.carekv_quantize_rows.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, vp]
        lib.carekv_prefill_attn.restype = C.c_int
        lib.carekv_prefill_attn.argtypes = [C.POINTER(PrefillParams), vp, vp, vp, vp, vp, vp]
        lib.carekv_dequantize_rows.restype = C.c_int
        lib.carekv_dequantize_rows.argtypes = [vp, vp, i32, i32, i32, vp, vp]
        lib.carekv_prefill_correct_workspace_bytes.restype = i64
        lib.carekv_prefill_correct_workspace_bytes.argtypes = [C.POINTER(Arena), C.POINTER(DecodeParams),
                                                               C.POINTER(PrefillCorrParams)]
        lib.carekv_prefill_correct.restype = C.c_int
        lib.carekv_prefill_correct.argtypes = [C.POINTER(Arena), C.POINTER(DecodeParams),
                                               C.POINTER(PrefillCorrParams), vp, vp, vp, i64, vp, i32, vp]
        lib.carekv_write_base.restype = C.c_int
        lib.carekv_write_base.argtypes = [C.POINTER(Arena), i32, i32, i32, vp, vp, vp, vp, i32, vp]
        for nm in ("carekv_pack_codes", "carekv_unpack_codes"):
            getattr(lib, nm).restype = C.c_int
            getattr(lib, nm).argtypes = [vp, i64, i32, i32, vp, vp]
        lib.carekv_pack_4bit.restype = C.c_int
        lib.carekv_pack_4bit.argtypes = [vp, i32, i64, vp, vp, vp]
        lib.carekv_unpack_4bit.restype = C.c_int
        lib.carekv_unpack_4bit.argtypes = [vp, vp, i64, vp, vp]
        lib.carekv_quantize_rows_f32.restype = C.c_int
        lib.carekv_quantize_rows_f32.argtypes = [vp, i64, i32, i32, i32, vp, vp, vp]
        lib.carekv_dequantize_rows_f32.restype = C.c_int
        lib.carekv_dequantize_rows_f32.argtypes = [vp, vp, i64, i32, i32, vp, vp]
        lib.carekv_kivi_qdq.restype = C.c_int
        lib.carekv_kivi_qdq.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp]
        lib.carekv_kivi_codes.restype = C.c_int
        lib.carekv_kivi_codes.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, vp]
        lib.carekv_read_hat_pages.restype = C.c_int
        lib.carekv_read_hat_pages.argtypes = [C.POINTER(Arena), i32, i32, i32, vp, vp, vp, vp, vp]
        lib.carekv_prefill_eval.restype = C.c_int
        lib.carekv_prefill_eval.argtypes = [C.POINTER(PrefillEvalParams), vp, vp, vp, vp, vp, vp, vp, vp, vp]
        _lib = lib
        return lib


def check(rc: int, what: str):
    if rc != 0:
        msg = load().carekv_last_error()
        raise CarekvError(f"{what} failed (code {rc}): {msg.decode() if msg else ''}")


def store_workspace_bytes(lib, arena, sp, n_jobs: int) -> int:
    """carekv_store_workspace_bytes for a call with this arena, these store
    params and n_jobs page jobs (raises on an invalid argument)."""
    n = int(lib.carekv_store_workspace_bytes(arena, sp, int(n_jobs)))
    if n < 0:
        check(-1, "carekv_store_workspace_bytes")
    return n


def check_enabled() -> bool:
    """CAREKV_CHECK=1: after each launch, read the call's status word back
    (a device-to-host copy, which waits for the stream) and raise on an
    overflow the kernels flagged.  Off by default: the hot path never syncs."""
    return os.environ.get("CAREKV_CHECK", "0") == "1"


def check_status(ws: torch.Tensor, index: int, what: str):
    """Raise if the int32 status word at ``index`` of the workspace is set."""
    flag = int(ws[4 * index:4 * index + 4].view(torch.int32).item())
    if flag != 0:
        raise CarekvError(f"{what}: the kernels flagged an overflow (status {flag}): a page holds more stored "
                          "residual slots than the record capacity (k_cap / v_cap), or a slot id fell past the "
                          "arena's n_slots; those slots were left out")


class StatusWatch:
    """Reports the store calls' status words without waiting for the
    stream: each word is copied to pinned host memory behind an event, and a
    later call (or ``poll``) warns, once per call site, about a word that was
    set (slot ids past the arena's n_slots, whose residuals were dropped)."""

    def __init__(self, n: int = 64):
        self.host = None
        self.n = n
        self.pending = collections.deque()  # (host index, event, what)
        self.next = 0
        self.warned = set()
        self.flagged = 0

    def watch(self, ws: torch.Tensor, index: int, what: str):
        self.poll()
        if self.host is None:
            self.host = torch.zeros(self.n, dtype=torch.int32, pin_memory=True)
        if len(self.pending) == self.n:
            self.pending[0][1].synchronize()
            self.poll()
        i = self.next
        self.next = (self.next + 1) % self.n
        self.host[i:i + 1].copy_(ws[4 * index:4 * index + 4].view(torch.int32), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.pending.append((i, ev, what))

    def poll(self, wait: bool = False) -> int:
        """Check the landed words (all of them with ``wait``); returns how
        many set words were seen so far."""
        while self.pending and (wait or self.pending[0][1].query()):
            i, ev, what = self.pending.popleft()
            ev.synchronize()
            if int(self.host[i]) != 0:
                self.flagged += 1
                if what not in self.warned:
                    self.warned.add(what)
                    warnings.warn(f"{what}: residual slot ids fell past the arena's n_slots and those slots were "
                                  "dropped; size the cache with a larger n_slots", RuntimeWarning, stacklevel=3)
        return self.flagged


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise CarekvError("CARE-KV HIP kernels need device tensors (got a CPU tensor); "
                          "there is no CPU implementation in the product path")
    return t.data_ptr()


def stream_ptr(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
