"""ctypes binding of librwkvq_hip.so (the C ABI declared in
include/rwkvq_hip.h).

The library is built in-tree by `rwkv-quant_amd/build_hip.py`; there is no
fallback: if it is missing or a call fails, an exception is raised.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RWKVQ_HIP_LIB",
                          os.path.join(_HERE, "librwkvq_hip.so"))

RWKVQ_OK = 0
ERRORS = {1001: "invalid argument or shape", 1002: "kernel launch failed",
          1003: "size beyond a supported limit"}

EPI_STORE, EPI_ADD, EPI_RELU2, EPI_TANH, EPI_SIGMOID = 0, 1, 2, 3, 4
EPI_PER_SEG = 5                # rwkvq_gemm_f16: mode per input segment
X_F16 = 16                     # GEMM flag: x is fp16 in the format's pair order
Y_F16 = 32                     # GEMM flag: y is fp16 in pair order (bits 6-7)
Y_ORDER_SHIFT = 6
NO_SPLIT = 256                 # GEMM flag: no split-K (concurrent streams)
ORDER_PAIRS, ORDER_SB6, ORDER_SYM6 = 0, 1, 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_long

# name -> argument types (all return int status)
SIGNATURES = {
    "rwkvq_gemv_sb6": [_P, _P, _P, _I, _I, _I, _I, _P, _L, _P, _I, _I, _P],
    "rwkvq_gemv_sym": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _L, _P, _I, _I,
                       _P],
    "rwkvq_gemv_rtn8": [_P, _P, _I, _I, _I, _P, _L, _P, _I, _I, _P],
    "rwkvq_gemv_rtn8_spqr": [_P, _P, _P, _P, _P, _I, _I, _P, _L, _P, _I, _I,
                             _P],
    "rwkvq_spqr_apply": [_P, _L, _P, _P, _P, _I, _I, _P, _I, _P],
    "rwkvq_spqr_scatter": [_P, _P, _P, _I, _P, _L, _P],
    "rwkvq_gemm_sb6": [_P, _P, _P, _I, _I, _I, _I, _P, _L, _P, _I, _I, _P],
    "rwkvq_gemm_sym": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _L, _P, _I, _I,
                       _P],
    "rwkvq_gemm_rtn8": [_P, _P, _I, _I, _I, _P, _L, _P, _I, _I, _P],
    "rwkvq_gemm_f16": [_P, _I, _I, _I, _P, _L, _P, _I, _I, _I, _P],
    "rwkvq_gemv_f16_seg": [_P, _I, _P, _I, _P, _L, _P, _I, _I, _P],
    "rwkvq_gemm_f16_seg": [_P, _I, _P, _I, _P, _L, _P, _I, _I, _I, _P],
    "rwkvq_gemm_workspace": [_P, _L, _P, _I],
    "rwkvq_gemm_plan": [_I, _I, _I, _I, _I, _P],
    "rwkvq_gemm_f16_grouped": [_I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rwkvq_gemm_dual_f16seg": [_I, _I, _P, _P, _P, _P, _I, _I, _I, _P, _L, _P,
                               _I, _P, _I, _P, _P, _L, _P, _I, _I, _I, _P],
    "rwkvq_x16": [_P, _L, _I, _I, _I, _P, _L, _P],
    "rwkvq_dequant_sb6_f32": [_P, _P, _P, _I, _I, _I, _P, _I, _P],
    "rwkvq_dequant_sym_f32": [_P, _P, _P, _P, _I, _I, _I, _P, _I, _P],
    "rwkvq_dequant_rtn8_f32": [_P, _P, _I, _I, _P, _I, _P],
    "rwkvq_dequant_asym_f32": [_P, _P, _P, _I, _I, _I, _P, _I, _P],
    "rwkvq_probe_stream_read": [_P, ctypes.c_long, _P, _I, _P],
    "rwkvq_nll_rows": [_P, _L, _P, _I, _I, _P, _P],
    "rwkvq_dequant_f16": [_I, _P, _P, _P, _P, _P, _I, _I, _P, _I, _P],
    "rwkvq_gather_rows_f32": [_I, _I, _P, _P, _P, _P, _I, _I, _P, _I, _P,
                              _P],
    "rwkvq_gather_ln_f32": [_I, _I, _P, _P, _P, _P, _I, _I, _P, _I, _P, _P,
                            _F, _P, _P],
    "rwkvq_layer_norm": [_P, _P, _P, _P, _I, _I, _F, _P],
    "rwkvq_shift_lerp": [_P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _P],
    "rwkvq_shift_lerp_f16": [_P, _P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                             _P],
    "rwkvq_wkv_prep": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P,
                       _P, _P, _P, _I, _I, _I, _P],
    "rwkvq_wkv7_scan": [_P, _L, _P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _I,
                        _I, _I, _I, _P],
    "rwkvq_wkv7_scan_chunked": [_P, _L, _P, _P, _P, _P, _P, _L, _P, _P, _P,
                                _L, _I, _I, _I, _I, _P, _L, _P],
    "rwkvq_wkv7_scan_chunked_noalloc": [_P, _L, _P, _P, _P, _P, _P, _L, _P,
                                        _P, _P, _L, _I, _I, _I, _I, _P],
    "rwkvq_wkv7_prefill_chunked": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _I, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                                   _P, _L, _P],
    "rwkvq_wkv_tail": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "rwkvq_wkv_tail_f16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                           _I, _P],
    "rwkvq_lora_gemv": [_I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P],
    "rwkvq_wkv7_decode_lora": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _P, _P, _I, _P, _P, _P, _I, _I, _I, _P],
    "rwkvq_wkv7_decode": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                          _P, _P, _I, _P, _P, _P, _I, _I, _I, _P],
    "rwkvq_lora_down_q": [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                          _P],
    "rwkvq_wkv7_decode_lora_q": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                 _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I,
                                 _I, _P],
    "rwkvq_decode_mk": [_P, _I, _I, _I, _I, _I, _I, _P, _P, _L, _P, _P, _P,
                        _P],
    "rwkvq_decode_mk_info": [_P, _P, _P, _P],
    "rwkvq_decode_mk_spin_limit": [_I],
}

_lib = None


class HipKernelError(RuntimeError):
    pass


def load():
    """Load the library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipKernelError(
            f"{LIB_PATH} is missing: build it with "
            f"`python rwkv-quant_amd/build_hip.py` (hipcc, gfx950)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    _lib = lib
    return lib


# split-K workspace of the GEMMs: partial tiles + arrival counters (zeroed
# once; every launch leaves them at zero)
GEMM_WS_BYTES = 64 << 20
GEMM_WS_COUNTERS = 8192
_gemm_ws = {}


def ensure_gemm_workspace():
    """Register the GEMM split-K workspace of the current device once
    (eagerly: never from inside a stream capture, where the GEMMs then run
    without splitting)."""
    import torch
    dev = torch.cuda.current_device()
    if dev in _gemm_ws or torch.cuda.is_current_stream_capturing():
        return
    ws = torch.empty(GEMM_WS_BYTES, dtype=torch.uint8, device=f"cuda:{dev}")
    cnt = torch.zeros(GEMM_WS_COUNTERS, dtype=torch.int32,
                      device=f"cuda:{dev}")
    torch.cuda.synchronize(dev)
    st = load().rwkvq_gemm_workspace(ptr(ws), GEMM_WS_BYTES, ptr(cnt),
                                     GEMM_WS_COUNTERS)
    if st != RWKVQ_OK:
        raise HipKernelError(f"rwkvq_gemm_workspace: status {st}")
    _gemm_ws[dev] = (ws, cnt)


def call(name, *args):
    """Invoke an entry point; a non-zero status raises HipKernelError."""
    if len(args) != len(SIGNATURES[name]):
        # ctypes would pass extra arguments on (as to a varargs function)
        raise TypeError(f"{name}: {len(args)} arguments, the C entry point "
                        f"takes {len(SIGNATURES[name])}")
    if name.startswith(("rwkvq_gemm_", "rwkvq_gemv_")) and \
            name != "rwkvq_gemm_workspace":
        # the GEMMs and the batched GEMV split K through the workspace
        # (rwkvq_gemm_plan too: the plan depends on it)
        ensure_gemm_workspace()
    st = getattr(load(), name)(*args)
    if st != RWKVQ_OK:
        raise HipKernelError(f"{name}: status {st} "
                             f"({ERRORS.get(st, 'hip error')})")


def gemm_plan(rows, in_features, out_per, M, mode=0):
    """The tile plan of a quantized GEMM (rwkvq_gemm_plan) as a dict."""
    out = (ctypes.c_int * 6)()
    call("rwkvq_gemm_plan", rows, in_features, out_per, M, mode, out)
    return dict(zip(("tile_rows", "tile_tokens", "waves", "kgroups",
                     "split", "workgroups"), list(out)))


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
