"""
ctypes binding of ``libmace_hip.so`` (declared in ``include/mace_hip.h``).

The library is built in-tree (``__graft_entry__.build()``) next to this file.  It must be loaded after torch so that
its ``libamdhip64.so.7`` / ``libhiprtc.so.7`` dependencies resolve to the copies torch already mapped; ``load()``
verifies that.  There is no fallback: a missing or broken library raises.
"""
import ctypes
import hashlib
import os
import re
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libmace_hip.so')
DEVICE_HEADER = os.path.join(os.path.dirname(HERE), 'csrc', 'mh_device.h')

MH_CONV_FWD, MH_CONV_BWD, MH_CONV_BWD_WY, MH_SC_FWD, MH_SC_BWD, MH_CONV_BWD_R, MH_CONV_GXSUM, MH_SC_FWD_G, \
    MH_SC_BWD_G, MH_CONV_BWD_RC, MH_CONV_FWD_C, MH_SH_FWD, MH_SH_BWD, MH_LIN_FWD, MH_LIN_BWD, \
    MH_MLP_FWD, MH_MLP_BWD, MH_EMB_FWD, MH_EMB_BWD, MH_PERM_FWD, MH_PERM_BWD, MH_GEOM_FWD, MH_GEOM_BWD, \
    MH_SC_FWD_I, MH_SC_BWD_I, MH_SC_FWD_GI, MH_SC_BWD_GI, MH_READOUT_FWD, MH_READOUT_BWD, MH_SC_JVP, MH_SC_BWD2, \
    MH_SC_JVP_I, MH_SC_BWD2_I, MH_CSR_FILL, MH_CSR_COUNT, MH_CSR_SCAN, MH_CSR_SCATTER, MH_CSR_RANK, MH_SH_JVP, \
    MH_SH_BWD2, MH_EMB_JVP, MH_EMB_BWD2, MH_GEOM_JVP, MH_READOUT_JVP, MH_READOUT_BWD2, MH_CSR_SORT, MH_MLP_HID, \
    MH_MLP_HIDB, MH_CONV_FWD_M, MH_CONV_BWD_M, MH_CONV_GYSUM, MH_SC_FWD_S, MH_SC_BWD_S, MH_SC_FWD_SI, \
    MH_SC_BWD_SI, MH_NL_SETUP, MH_NL_ZERO, MH_NL_BINS, MH_NL_SCAN, MH_NL_PLACE, MH_NL_COUNT, MH_NL_OFFSETS, \
    MH_NL_FILL, MH_SPECIES_ORDER, MH_MLP_JVP, MH_MLP_BWD2, MH_GEOM_SEGSUM, MH_NL_BASES, MH_EDGE_COUNT, \
    MH_EDGE_PLACE, MH_GEOM_SEGSUM1, MH_EDGE_PAIR, MH_CONV_FWD_CR, MH_MLP_H3, MH_MLP_OUT, MH_EDGE_FWD, \
    MH_EDGE_BWD, MH_MLP_BWD_P, MH_LIN_BWD_SUM = range(79)
MH_WANT_GX, MH_WANT_GWY, MH_CUT_MASKED, MH_CUT_NOZERO = 1, 2, 4, 8
ABI_VERSION = 42

# hipcc/hipRTC options for every generated layer: gfx950 code, -O3, and packed-FP32 instructions disabled.
ARCH = os.environ.get('MACE_HIP_ARCH', 'gfx950')
COMPILE_OPTIONS = f'--offload-arch={ARCH} -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops'

_lib = None
_lock = threading.Lock()
_code_cache = {}

_P = ctypes.c_void_p
_I = ctypes.c_int32
_SIGS = {
    'mh_last_error': (ctypes.c_char_p, []),
    'mh_version': (ctypes.c_int, []),
    'mh_hip_runtime_path': (ctypes.c_char_p, []),
    'mh_compile': (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_size_t)]),
    'mh_free_code': (None, [_P]),
    'mh_module_load': (ctypes.c_int, [_P, ctypes.c_size_t, ctypes.POINTER(_P)]),
    'mh_module_unload': (ctypes.c_int, [_P]),
    'mh_module_bind': (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.c_int]),
    'mh_conv_fwd': (ctypes.c_int, [_P] * 8 + [_I, _P]),
    'mh_conv_bwd_x': (ctypes.c_int, [_P] * 8 + [_I, _P]),
    'mh_conv_bwd_wy': (ctypes.c_int, [_P] * 9 + [_I, _P]),
    'mh_conv_bwd': (ctypes.c_int, [_P] * 11 + [_I, _I, _P]),
    'mh_conv_bwd_recv': (ctypes.c_int, [_P] * 16 + [_I, _I, _P]),
    'mh_conv_fwd_cut': (ctypes.c_int, [_P] * 9 + [_I, _P]),
    'mh_conv_bwd_recv_rows': (ctypes.c_int, [_P] * 17 + [_I, _I, _P]),
    'mh_conv_fwd_cut_rows': (ctypes.c_int, [_P] * 10 + [_I, _P]),
    'mh_sh_fwd': (ctypes.c_int, [_P] * 3 + [ctypes.c_int64, _P]),
    'mh_sh_bwd': (ctypes.c_int, [_P] * 4 + [ctypes.c_int64, _P]),
    'mh_lin_fwd': (ctypes.c_int, [_P] * 6 + [ctypes.c_float, ctypes.c_int, _P]),
    'mh_lin_bwd': (ctypes.c_int, [_P] * 6 + [ctypes.c_float, ctypes.c_int, _P]),
    'mh_lin_fwd_res': (ctypes.c_int, [_P] * 6 + [ctypes.c_float, _P, ctypes.c_int, _P]),
    'mh_lin_bwd_sum': (ctypes.c_int, [_P] * 8 + [ctypes.c_float, ctypes.c_int, _P]),
    'mh_readout_fwd': (ctypes.c_int, [_P] * 3 + [ctypes.c_int64, _P]),
    'mh_readout_bwd': (ctypes.c_int, [_P] * 4 + [ctypes.c_int64, _P]),
    'mh_mlp_fwd': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_mlp_bwd': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P]),
    'mh_mlp_fwd_rows': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P, _P, _P]),
    'mh_mlp_fwd_ws': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P, _P, ctypes.c_int32, _P]),
    'mh_mlp_bwd_rows': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P, _P, _P]),
    'mh_mlp_bwd_pairs': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P, _P, _P, _P]),
    'mh_edge_compact_work_size': (ctypes.c_size_t, [ctypes.c_int64]),
    'mh_geom_segsum1': (ctypes.c_int, [_P, _P, _P, _P, _I, _P]),
    'mh_edge_compact': (ctypes.c_int, [_P, _P, ctypes.c_int64, _P, _P, _P, _P]),
    'mh_edge_pairs_work_size': (ctypes.c_size_t, [ctypes.c_int64]),
    'mh_edge_pairs': (ctypes.c_int, [_P, _P, _I] + [_P] * 7 + [_I, ctypes.c_int64] + [_P] * 9),
    'mh_emb_fwd': (ctypes.c_int, [_P] * 4 + [ctypes.c_int64, _P]),
    'mh_emb_bwd': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_edge_fwd': (ctypes.c_int, [_P] * 10 + [ctypes.c_int64, _P]),
    'mh_edge_bwd': (ctypes.c_int, [_P] * 8 + [ctypes.c_int64, _P]),
    'mh_edge_bwd2': (ctypes.c_int, [_P] * 11 + [ctypes.c_int64, _P]),
    'mh_perm_fwd': (ctypes.c_int, [_P] * 3 + [ctypes.c_int, _P]),
    'mh_perm_bwd': (ctypes.c_int, [_P] * 3 + [ctypes.c_int, _P]),
    'mh_geom_fwd': (ctypes.c_int, [_P] * 7 + [ctypes.c_int64, _P]),
    'mh_geom_bwd': (ctypes.c_int, [_P] * 11 + [ctypes.c_int, _P]),
    'mh_module_bind_grid': (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    'mh_sc_fwd_sorted': (ctypes.c_int, [_P] * 6 + [_I, _P]),
    'mh_sc_fwd_irreps': (ctypes.c_int, [_P] * 6 + [_I, _P]),
    'mh_sc_bwd_irreps': (ctypes.c_int, [_P] * 7 + [_I, _P]),
    'mh_sc_fwd_staged': (ctypes.c_int, [_P] * 3 + [_I] + [_P] * 3 + [_I, _I, _P]),
    'mh_sc_bwd_staged': (ctypes.c_int, [_P] * 3 + [_I] + [_P] * 4 + [_I, _I, _P]),
    'mh_sc_bwd_sorted': (ctypes.c_int, [_P] * 7 + [_I, _P]),
    'mh_sc_fwd': (ctypes.c_int, [_P] * 5 + [_I, _P]),
    'mh_sc_jvp': (ctypes.c_int, [_P] * 6 + [_I, _I, _P]),
    'mh_graph_build': (ctypes.c_int, [_P, _P, ctypes.c_int64, _I] + [_P] * 6),
    'mh_graph_build_noalloc': (ctypes.c_int, [_P, _P, ctypes.c_int64, _I] + [_P] * 5),
    'mh_mlp_hid': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_mlp_hid_bwd': (ctypes.c_int, [_P] * 4 + [_I] + [_P] * 3 + [ctypes.c_int64, _P]),
    'mh_conv_fwd_mlp': (ctypes.c_int, [_P] * 10 + [_I, _P]),
    'mh_conv_bwd_mlp': (ctypes.c_int, [_P] * 18 + [_I, _I, _I, _P]),
    'mh_launch_log': (ctypes.c_int, [ctypes.c_int]),
    'mh_launch_log_take': (ctypes.c_size_t, [ctypes.c_char_p, ctypes.c_size_t]),
    'mh_sh_jvp': (ctypes.c_int, [_P] * 4 + [ctypes.c_int64, _P]),
    'mh_sh_bwd2': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_emb_jvp': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_emb_bwd2': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P]),
    'mh_geom_jvp': (ctypes.c_int, [_P] * 11 + [ctypes.c_int64, _P]),
    'mh_readout_jvp': (ctypes.c_int, [_P] * 4 + [ctypes.c_int64, _P]),
    'mh_readout_bwd2': (ctypes.c_int, [_P] * 5 + [ctypes.c_int64, _P]),
    'mh_sc_bwd2': (ctypes.c_int, [_P] * 7 + [_I, _I, _P]),
    'mh_sc_bwd': (ctypes.c_int, [_P] * 6 + [_I, _P]),
    'mh_geom_segsum': (ctypes.c_int, [_P] * 5 + [_I, _P]),
    'mh_mlp_jvp': (ctypes.c_int, [_P] * 6 + [ctypes.c_int64, _P]),
    'mh_mlp_bwd2': (ctypes.c_int, [_P] * 7 + [ctypes.c_int64, _P]),
    'mh_species_order': (ctypes.c_int, [_P, _P, _I, _I, _P, _P, _P, _I, _I, _P]),
    'mh_neighbour_list_work_size': (ctypes.c_size_t, [_I, _I, ctypes.c_int64]),
    'mh_neighbour_list': (ctypes.c_int, [_P] * 5 + [_I, _I, ctypes.c_double, ctypes.c_int64, ctypes.c_int64]
                          + [_P] * 3 + [_I] + [_P] * 3),
}
EXPORTS = tuple(_SIGS)


def load():
    """The bound library (loaded once).  Raises if it is missing, stale or bound to a foreign HIP runtime."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f'mace_hip_kernels: {LIB_PATH} is missing; build it with __graft_entry__.build()')
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.mh_version() != ABI_VERSION:
            raise RuntimeError('mace_hip_kernels: libmace_hip.so ABI version mismatch; rebuild it')
        rt = lib.mh_hip_runtime_path().decode()
        torch_lib = os.path.realpath(os.path.join(os.path.dirname(torch.__file__), 'lib'))
        if rt and os.path.dirname(os.path.realpath(rt)) != torch_lib:
            raise RuntimeError(f'mace_hip_kernels: libmace_hip.so bound HIP runtime {rt}, not the one torch loaded '
                               f'from {torch_lib}; import torch before mace_hip_kernels')
        _lib = lib
    return _lib


def check(rc, what=''):
    if rc != 0:
        msg = load().mh_last_error().decode(errors='replace')
        raise RuntimeError(f'mace_hip_kernels: {what} failed (code {rc}): {msg}')


def device_header():
    with open(DEVICE_HEADER) as f:
        return f.read()


def dual_header():
    """Forward-mode dual numbers (``mh_dual``) for the second-order kernels."""
    with open(os.path.join(os.path.dirname(DEVICE_HEADER), 'mh_dual.h')) as f:
        return f.read()


def dualize(lines):
    """C statements with every ``float`` declared as ``mh_dual`` (the same arithmetic carried on dual numbers)."""
    return [re.sub(r'\bfloat\b', 'mh_dual', l) for l in lines]


def compile_source(source):
    """hipRTC-compile ``source`` → code-object bytes (cached per process by source hash; no GPU needed)."""
    key = hashlib.sha256((COMPILE_OPTIONS + '\0' + source).encode()).hexdigest()
    if key in _code_cache:
        return _code_cache[key]
    lib = load()
    code, size = _P(), ctypes.c_size_t()
    check(lib.mh_compile(source.encode(), COMPILE_OPTIONS.encode(), ctypes.byref(code), ctypes.byref(size)),
          'hipRTC compile')
    try:
        data = ctypes.string_at(code, size.value)
    finally:
        lib.mh_free_code(code)
    _code_cache[key] = data
    return data


class Module:
    """A loaded per-layer code object with its kernels bound to launch slots (owned; unloaded on deletion)."""

    def __init__(self, code, kernels):
        lib = load()
        self._lib = lib
        self.handle = _P()
        self._code = code
        buf = ctypes.create_string_buffer(code, len(code))
        check(lib.mh_module_load(buf, len(code), ctypes.byref(self.handle)), 'module load')
        self.device = torch.cuda.current_device()
        for kind, (name, block, rows, *grid_y) in kernels.items():
            check(lib.mh_module_bind_grid(self.handle, kind, name.encode(), block, rows, grid_y[0] if grid_y else 1),
                  f'bind {name}')

    def __del__(self):
        h = getattr(self, 'handle', None)
        if h is not None and h.value and getattr(self, '_lib', None) is not None:
            try:
                self._lib.mh_module_unload(h)
            except Exception:  # noqa: BLE001  (interpreter shutdown)
                pass


def launch_log_take():
    """Symbols of the kernels launched since the last call, oldest first (the C ABI's launch log)."""
    lib = load()
    n = lib.mh_launch_log_take(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib.mh_launch_log_take(buf, n + 1)
    return [s for s in buf.value.decode().split(';') if s]


class timing:
    """Context manager: while active, every kernel launch is bracketed by two HIP events recorded on the launch
    stream; ``.records`` collects (tag, start, end) and ``.symbols`` maps each tag to the kernel symbols its launches
    ran, as the C ABI's launch log recorded them.  Off by default (no events outside this context)."""
    active = None

    def __init__(self):
        self.records = []
        self.symbols = {}

    def __enter__(self):
        timing.active = self
        self._was = load().mh_launch_log(1)
        launch_log_take()
        return self

    def __exit__(self, *exc):
        timing.active = None
        load().mh_launch_log(self._was)

    def summary(self):
        """{tag: (launches, mean ms)} (synchronises the device)."""
        torch.cuda.synchronize()
        acc = {}
        for tag, s, e in self.records:
            n, tot = acc.get(tag, (0, 0.0))
            acc[tag] = (n + 1, tot + s.elapsed_time(e))
        return {k: (n, tot / n) for k, (n, tot) in acc.items()}


def launch(tag, fn, *args):
    """Call a C-ABI launcher, raise on a nonzero status, and time it when a ``timing`` context is active."""
    rec = timing.active
    if rec is None:
        check(fn(*args), tag)
        return
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    check(fn(*args), tag)
    e.record()
    rec.records.append((tag, s, e))
    syms = rec.symbols.setdefault(tag, [])
    for name in launch_log_take():
        if name not in syms:
            syms.append(name)


def ptr(t):
    """Device pointer of a tensor (None → NULL)."""
    return None if t is None else _P(t.data_ptr())


def stream_of(t):
    return _P(torch.cuda.current_stream(t.device).cuda_stream)


# ------------------------------------------------------------------------------------------- graph capture
# Device memory that a graph being captured reads but does not own (cached CSRs and element indices built by earlier
# eager calls).  A captured kernel node keeps raw pointers, so whoever owns the graph must keep these objects alive:
# ``graphs.capture`` takes them with ``take_capture_holds`` right after capture.
_capture_holds = []


def capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def hold_for_capture(obj):
    """Register ``obj`` as read by the graph being captured on the current stream (no-op outside capture)."""
    if capturing():
        _capture_holds.append(obj)
    return obj


def take_capture_holds():
    held = list(_capture_holds)
    _capture_holds.clear()
    return held
