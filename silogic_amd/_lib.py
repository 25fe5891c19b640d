"""ctypes binding of ``libsilogic_hip.so`` (declared in ``include/silogic_hip.h``).

The library is loaded from ``silogic_amd/lib`` (built in-tree by
``__graft_entry__.build()``) or from the path in ``SILOGIC_HIP_LIB``. There is
no fallback: if the library cannot be loaded, :func:`lib` raises and every
GPU forward of the package raises with it.
"""
import ctypes as C
import os
import threading

from . import _build

_P, _I32, _I64, _F32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float

# name -> (restype, argtypes); mirrors include/silogic_hip.h one to one
SIGNATURES = {
    "slg_last_error": (C.c_char_p, []),
    "slg_version": (C.c_int, []),
    "slg_device_cus": (C.c_int, []),
    "slg_dense_logic_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "slg_warp_logic_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _F32, _P, _P]),
    "slg_fc_soft_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _P, _I32, _P, _F32, _P, _I32,
                                  _I32, _P]),
    "slg_fc_soft_prep": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "slg_fc_soft_records": (C.c_int, [_I32, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P]),
    "slg_fc_soft_schedule": (C.c_int, [_P, _I64, _I32, _I64, _P, _P]),
    "slg_fc_soft_fwd_records": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _I64, _I32, _F32, _P,
                                          _I32, _I32, _P]),
    "slg_fc_soft_fwd_groupsum": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _I64, _I32, _F32,
                                           _I32, _F32, _P, _P]),
    "slg_fc_soft_groupsum_supported": (C.c_int, [_I64, _I64, _I64, _I32]),
    "slg_fc_soft_net_supported": (C.c_int, [_I64, _I64, _I32, _P, _I32, _I32]),
    "slg_fc_soft_net_records": (C.c_int, [_P, _I64, _I64, _I32, _P, _P, _P, _I32, _I32, _F32, _I32,
                                          _F32, _P, _P]),
    "slg_groupsum_soft": (C.c_int, [_P, _I64, _I64, _I32, _F32, _I32, _P, _P]),
    "slg_groupsum_hard": (C.c_int, [_P, _I32, _I64, _I64, _I32, _P, _P]),
    "slg_orpool": (C.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "slg_pack_bits": (C.c_int, [_P, _I32, _I64, _I64, _I32, _P, _P]),
    "slg_unpack_bits": (C.c_int, [_P, _I64, _I64, _P, _P]),
    "slg_fc_hard_prep": (C.c_int, [_P, _P, _I64, _I32, _I64, _I32, _P, _P, _P]),
    "slg_fc_hard_prep_net": (C.c_int, [_I32, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P]),
    "slg_fc_hard_layer": (C.c_int, [_P, _I64, _I64, _P, _I64, _P, _P]),
    "slg_fc_hard_net": (C.c_int, [_P, _I32, _I64, _I64, _I32, _P, _P, _I32, _I64, _P, _P]),
    "slg_fc_hard_place_net": (C.c_int, [_I32, _P, _P, _P, _P, _I64, _P]),
    "slg_fc_hard_type_slots": (C.c_int64, [_I64, _I32, _P]),
    "slg_fc_hard_type_place_workspace": (_I64, [_I32, _P]),
    "slg_fc_hard_type_place_net": (C.c_int, [_I32, _I64, _P, _P, _P, _P, _P, _I64, _P]),
    "slg_fc_hard_net_typed": (C.c_int, [_P, _I32, _I64, _I64, _I32, _P, _P, _P, _I32, _P, _P]),
    "slg_fc_hard_net_supported": (C.c_int, [_I64, _I32, _P, _I32]),
    "slg_groupsum_packed": (C.c_int, [_P, _I64, _I64, _I32, _P, _P]),
    "slg_fc_soft_bwd_workspace": (C.c_int64, [_I64, _I64, _I64, _I32]),
    "slg_fc_soft_bwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _P, _P, _I32, _P, _F32, _P, _P, _P, _P,
                                  _P, _I64, _P]),
    "slg_conv_soft_bwd_workspace": (C.c_int64, [_I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32,
                                                _I32, _I32, _I32]),
    "slg_conv_soft_bwd": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P,
                                    _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _I64, _P]),
    "slg_fc_lut_soft_workspace": (C.c_int64, [_I64, _I32, _I32]),
    "slg_fc_lut_soft_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _I32, _P, _P,
                                      _I64, _P]),
    "slg_fc_lut_soft_fwd_noalloc": (C.c_int, [_P, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _I32,
                                              _P, _P]),
    "slg_fc_lut_soft_bwd_workspace": (C.c_int64, [_I64, _I64, _I64, _I32, _I32]),
    "slg_fc_lut_soft_bwd": (C.c_int, [_P, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P,
                                      _P, _P, _I64, _P]),
    "slg_fc_lut_hard_prep": (C.c_int, [_P, _P, _I64, _I32, _I32, _I64, _P, _P, _P, _P]),
    "slg_encode_thermometer": (C.c_int, [_P, _I32, _I64, _I64, _P, _I32, _I32, _I32, _P, _P]),
    "slg_edge_bits": (C.c_int, [_P, _I64, _I64, _I64, _I64, _P, _I32, _P, _P]),
    "slg_learned_thermo_bwd_workspace": (C.c_int64, [_I64, _I64, _I32]),
    "slg_learned_thermo_bwd": (C.c_int, [_P, _I64, _I64, _I32, _P, _F32, _P, _P, _P, _P, _I64,
                                         _P]),
    "slg_fc_lut_hard": (C.c_int, [_P, _I64, _I64, _P, _I32, _P, _I64, _P, _P]),
    "slg_packed_unfold": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P]),
    "slg_packed_or_pool": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "slg_lut_tree_hard": (C.c_int, [_P, _I64, _I64, _I64, _I64, _P, _I32, _I32, _P, _P, _P]),
    "slg_tree_conv_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _P,
                                    _P, _I32, _I32, _I64, _I64, _P, _P]),
    "slg_conv_soft_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P,
                                    _P, _P, _P, _P, _I32, _I32, _P, _P]),
    "slg_conv_soft_prep": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "slg_conv_soft_lds_fit": (C.c_int, [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32]),
    "slg_conv_soft_record_floats": (C.c_int64, [_I32, _I32, _I32, _I32, _I32]),
    "slg_conv_soft_records": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _I64,
                                        _I64, _I64, _I32, _I32, _P, _P]),
    "slg_conv_soft_records_arrays": (C.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32,
                                               _I64, _I64, _I64, _I32, _I32, _P, _P]),
    "slg_conv_soft_fwd_records": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32,
                                            _I32, _P, _I32, _I32, _P, _P]),
    "slg_conv_hard_prep": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P,
                                     _P, _P]),
    "slg_conv_hard_prep_net": (C.c_int, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                         _P]),
    "slg_conv_tree_hard_prep": (C.c_int, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P,
                                          _P, _P]),
    "slg_conv_tree_hard_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P,
                                         _I32, _I32, _I32, _P, _P]),
    "slg_conv_hard_fwd": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P, _P,
                                    _I32, _I32, _I32, _P, _P]),
    "slg_hard_step": (C.c_int, [_P, _P, _P, _P]),
    "slg_conv_hard_fwd_wm": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P,
                                       _P, _I32, _I32, _P, _I32, _P]),
    "slg_pack_image_wm": (C.c_int, [_P, _I32, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "slg_hard_step_fuses_head": (C.c_int, [_P]),
    "slg_conv_hard_head_wm": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P,
                                        _P, _I32, _I32, _I64, _P, _P, _I32, _P, _P]),
    "slg_conv_hard_net_wm": (C.c_int, [_P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P,
                                       _P, _I32, _I32, _I32, _P, _P, _P, _I32, _P, _P]),
}

_lock = threading.Lock()
_lib = None
_load_error = None


class StepConv(C.Structure):
    """``slg_step_conv_t``: one conv block of a ``slg_hard_step_t``."""
    _fields_ = [("inp", _P), ("out", _P), ("C", _I64), ("H", _I64), ("W", _I64), ("N", _I64),
                ("node_kind", _I32), ("depth", _I32), ("arity", _I32), ("kernel", _I32),
                ("pad", _I32), ("out_pad", _I32), ("leaf", _P), ("tt", _P)]


STEP_MAX_CONV = 8


class HardStep(C.Structure):
    """``slg_hard_step_t``: a network's forward_hard launch sequence."""
    _fields_ = [("pack", _I32), ("dtype", _I32), ("B", _I64), ("C", _I64), ("H", _I64),
                ("W", _I64), ("pack_pad", _I32), ("packed", _P), ("n_conv", _I32),
                ("conv", StepConv * STEP_MAX_CONV), ("head_in", _P), ("head_in_kind", _I32),
                ("head_in_dim", _I64), ("n_layers", _I32), ("widths", _P), ("codes", _P),
                ("plan", _P), ("n_classes", _I32), ("wire_r", _I64)]


def library_path():
    return os.environ.get("SILOGIC_HIP_LIB", _build.LIB)


def lib():
    """Load (once) and return the library; raise ``ImportError`` if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            _load_error = f"{path} not found: build it with __graft_entry__.build()"
            raise ImportError("silogic_amd HIP library unavailable: " + _load_error)
        try:
            h = C.CDLL(path)
        except OSError as e:
            _load_error = str(e)
            raise ImportError("silogic_amd HIP library failed to load: " + _load_error) from e
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(h, name)
            except AttributeError as e:
                _load_error = f"{path} lacks {name}: rebuild it with __graft_entry__.build()"
                raise ImportError("silogic_amd HIP library is stale: " + _load_error) from e
            fn.restype = res
            fn.argtypes = args
        _lib = h
        return _lib


def available():
    try:
        lib()
        return True
    except ImportError:
        return False


class HipError(RuntimeError):
    pass


def check(rc, what):
    if rc != 0:
        msg = lib().slg_last_error().decode(errors="replace")
        raise HipError(f"{what} failed (code {rc}): {msg}")


def call(name, *args):
    """Call entry point ``name``; raise :class:`HipError` on a non-zero code."""
    fn = getattr(lib(), name)
    check(fn(*args), name)
