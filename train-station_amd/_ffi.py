"""ctypes bindings of the two native libraries of this package.

``libts_hip.so``       -- the C-ABI of ``include/ts_hip.h`` (HIP kernels for gfx950)
``libts_gradtrack.so`` -- the C handle API of ``include/ts_gradtrack.h``

Both are built in place by ``make -C train-station_amd`` (or
``__graft_entry__.build()``).  There is no fallback: if a library is missing
or fails to load, importing the package raises.
"""
from __future__ import annotations

import ctypes
import pathlib

HERE = pathlib.Path(__file__).resolve().parent

_c = ctypes
F = _c.POINTER(_c.c_float)
SZ = _c.c_size_t
VP = _c.c_void_p
U64P = _c.POINTER(_c.c_ulonglong)


class TsError(RuntimeError):
    """A panic of the reference (or a HIP error) raised by the native library."""


def _load(name: str) -> ctypes.CDLL:
    path = HERE / name
    if not path.exists():
        raise ImportError(f"{path} is missing: build it with `make -C {HERE}` "
                          "or __graft_entry__.build(); there is no CPU fallback")
    return ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)


# --- include/ts_hip.h ------------------------------------------------------------

MAP_MAX_INPUTS, MAP_MAX_OPS, MAP_MAX_OUTPUTS, MAP_REGS = 5, 24, 4, 16
# TS_HIP_MAP_* op codes and flags of include/ts_hip.h
MAP_CODES = {"add": 0, "sub": 1, "mul": 2, "div": 3, "neg": 4, "relu": 5, "relu_bwd": 6, "add_s": 7, "sub_s": 8,
             "mul_s": 9, "div_s": 10, "square": 11}
MAP_CHECKED = 1


XF_MAX_OPS = 4
# TS_HIP_XF_* operand-transform op codes of include/ts_hip.h
XF_CODES = {"add_s": 0, "sub_s": 1, "mul_s": 2, "div_s": 3, "rsub_s": 4, "rdiv_s": 5, "relu": 6, "relu_bwd_s": 7,
            "square": 8}


class OperandXf(ctypes.Structure):
    """struct ts_hip_operand_xf of include/ts_hip.h"""
    _fields_ = [("n_ops", _c.c_uint32), ("code", _c.c_uint8 * XF_MAX_OPS), ("imm", _c.c_float * XF_MAX_OPS)]


class MapOp(ctypes.Structure):
    """struct ts_hip_map_op of include/ts_hip.h"""
    _fields_ = [("code", _c.c_uint8), ("a", _c.c_uint8), ("b", _c.c_uint8), ("flags", _c.c_uint8),
                ("imm", _c.c_float), ("d", _c.c_uint8)]


class MapProgram(ctypes.Structure):
    """struct ts_hip_map_program of include/ts_hip.h"""
    _fields_ = [("inputs", VP * MAP_MAX_INPUTS), ("scalar_inputs", _c.c_uint32), ("n_inputs", _c.c_uint32),
                ("n_ops", _c.c_uint32), ("n_outputs", _c.c_uint32), ("ops", MapOp * MAP_MAX_OPS),
                ("outputs", VP * MAP_MAX_OUTPUTS), ("output_regs", _c.c_uint8 * MAP_MAX_OUTPUTS),
                ("reduce_reg", _c.c_int32), ("const_inputs", _c.c_uint32),
                ("const_values", _c.c_float * MAP_MAX_INPUTS)]


# name -> (restype, argtypes); every symbol declared in include/ts_hip.h
HIP_SIGNATURES = {
    "ts_hip_initialize": (_c.c_int, []),
    "ts_hip_cleanup": (None, []),
    "ts_hip_get_device_count": (_c.c_int, [_c.POINTER(_c.c_int)]),
    "ts_hip_set_device": (_c.c_int, [_c.c_int]),
    "ts_hip_get_device": (_c.c_int, [_c.POINTER(_c.c_int)]),
    "ts_hip_malloc": (_c.c_int, [_c.POINTER(F), SZ]),
    "ts_hip_free": (_c.c_int, [F]),
    "ts_hip_memcpy": (_c.c_int, [VP, VP, SZ, _c.c_int]),
    "ts_hip_memcpy_async": (_c.c_int, [VP, VP, SZ, _c.c_int, VP]),
    "ts_hip_memcpy_bytes": (_c.c_int, [VP, VP, SZ, _c.c_int, VP]),
    "ts_hip_host_malloc": (_c.c_int, [_c.POINTER(VP), SZ]),
    "ts_hip_host_free": (_c.c_int, [VP]),
    "ts_hip_stream_create": (_c.c_int, [_c.POINTER(VP)]),
    "ts_hip_stream_destroy": (_c.c_int, [VP]),
    "ts_hip_stream_synchronize": (_c.c_int, [VP]),
    "ts_hip_device_synchronize": (_c.c_int, []),
    "ts_hip_event_create": (_c.c_int, [_c.POINTER(VP)]),
    "ts_hip_event_destroy": (_c.c_int, [VP]),
    "ts_hip_event_record": (_c.c_int, [VP, VP]),
    "ts_hip_event_synchronize": (_c.c_int, [VP]),
    "ts_hip_event_elapsed_ms": (_c.c_int, [_c.POINTER(_c.c_float), VP, VP]),
    "ts_hip_timing_begin": (_c.c_int, [VP, VP]),
    "ts_hip_timing_end": (_c.c_int, [_c.POINTER(_c.c_int)]),
    "ts_hip_error_string": (_c.c_char_p, [_c.c_int]),
    "ts_hip_mem_info": (_c.c_int, [_c.POINTER(SZ), _c.POINTER(SZ)]),
    "ts_hip_add": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_sub": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_mul": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_div": (_c.c_int, [VP, VP, VP, SZ, SZ, VP, VP]),
    "ts_hip_add_scalar": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_sub_scalar": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_mul_scalar": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_div_scalar": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_neg": (_c.c_int, [VP, VP, SZ, SZ, VP]),
    "ts_hip_relu": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_pow_scalar": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_bias_add": (_c.c_int, [VP, VP, VP, SZ, SZ, _c.c_int, VP]),
    "ts_hip_row_broadcast": (_c.c_int, [_c.c_int, VP, VP, VP, SZ, SZ, _c.c_int, SZ, VP, VP]),
    "ts_hip_fill": (_c.c_int, [VP, _c.c_float, SZ, VP]),
    "ts_hip_randn": (_c.c_int, [VP, SZ, _c.c_uint64, VP]),
    "ts_hip_encode_f32_records": (_c.c_int, [VP, SZ, VP, VP]),
    "ts_hip_decode_f32_records": (_c.c_int, [VP, SZ, VP, VP, VP]),
    "ts_hip_fill_from_device": (_c.c_int, [VP, VP, _c.c_float, _c.c_int, SZ, VP]),
    "ts_hip_copy": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_relu_backward": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_pow_backward": (_c.c_int, [VP, VP, VP, SZ, _c.c_float, VP]),
    "ts_hip_mul_backward": (_c.c_int, [VP, VP, VP, VP, VP, SZ, VP]),
    "ts_hip_div_backward": (_c.c_int, [VP, VP, VP, VP, VP, SZ, SZ, SZ, VP, VP]),
    "ts_hip_exp": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_log": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_tanh": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_sqrt": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_sigmoid": (_c.c_int, [VP, VP, SZ, VP]),
    "ts_hip_leaky_relu": (_c.c_int, [VP, _c.c_float, VP, SZ, VP]),
    "ts_hip_softmax": (_c.c_int, [VP, VP, SZ, SZ, SZ, VP]),
    "ts_hip_broadcast_copy": (_c.c_int, [VP, _c.POINTER(SZ), SZ, VP, _c.POINTER(SZ), SZ, _c.c_float,
                                         _c.c_int, VP]),
    "ts_hip_reduce_sum": (_c.c_int, [VP, _c.POINTER(SZ), SZ, _c.c_uint, VP, _c.c_float, _c.c_int, VP]),
    "ts_hip_transpose": (_c.c_int, [VP, _c.POINTER(SZ), SZ, SZ, SZ, VP, VP]),
    "ts_hip_map_jit_mode": (_c.c_int, [_c.c_int]),
    "ts_hip_map_jit_stats": (_c.c_int, [_c.POINTER(SZ), _c.POINTER(SZ)]),
    "ts_hip_map_jit_log": (_c.c_char_p, []),
    "ts_hip_map_jit_source": (SZ, [VP, _c.c_int, _c.c_char_p, SZ]),
    "ts_hip_log_backward": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_sqrt_backward": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_tanh_backward": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_sigmoid_backward": (_c.c_int, [VP, VP, VP, SZ, VP]),
    "ts_hip_leaky_relu_backward": (_c.c_int, [VP, VP, VP, SZ, _c.c_float, VP]),
    "ts_hip_softmax_backward": (_c.c_int, [VP, VP, VP, SZ, SZ, SZ, VP]),
    "ts_hip_sum_workspace_floats": (SZ, [SZ]),
    "ts_hip_map_workspace_floats": (SZ, [SZ]),
    "ts_hip_map": (_c.c_int, [_c.POINTER(MapProgram), SZ, SZ, SZ, VP, VP, _c.c_int, VP, SZ, VP]),
    "ts_hip_sum": (_c.c_int, [VP, SZ, VP, VP, SZ, VP]),
    "ts_hip_mean": (_c.c_int, [VP, SZ, VP, VP, SZ, VP]),
    "ts_hip_sum_dim0_workspace_floats": (SZ, [SZ, SZ]),
    "ts_hip_sum_dim0": (_c.c_int, [VP, SZ, SZ, VP, VP, SZ, VP]),
    "ts_hip_matmul": (_c.c_int, [VP, VP, VP, SZ, SZ, SZ, VP]),
    "ts_hip_gemm": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, SZ, VP]),
    "ts_hip_gemm_fused": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, _c.c_int, VP, VP, SZ,
                                     VP, SZ, VP]),
    "ts_hip_gemm_noalloc": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, SZ, VP]),
    "ts_hip_gemm_colsum_workspace_floats": (SZ, [_c.c_int, SZ, SZ, SZ]),
    "ts_hip_gemm_colsum": (_c.c_int, [_c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, SZ, VP, VP, SZ, VP]),
    "ts_hip_gemm_takes_xf": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, _c.c_int]),
    "ts_hip_launch_group_begin": (_c.c_int, [VP]),
    "ts_hip_launch_group_end": (_c.c_int, [VP]),
    "ts_hip_gemm_takes_bsum": (_c.c_int, [_c.c_int, SZ, SZ, SZ]),
    "ts_hip_gemm_colsum_bsum": (_c.c_int, [_c.c_int, SZ, SZ, SZ, VP, SZ, VP, VP, VP, VP, SZ, VP, VP, VP,
                                           _c.c_int, VP]),
    "ts_hip_gemm_takes_sub": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ]),
    "ts_hip_gemm_fused_sub": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, VP, _c.c_int, VP, VP,
                                         SZ, VP]),
    "ts_hip_gemm_fused_xf": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, VP, SZ, VP, VP, _c.c_int, VP,
                                        VP, SZ, VP, SZ, VP]),
    "ts_hip_gemm_colsum_xf": (_c.c_int, [_c.c_int, SZ, SZ, SZ, VP, SZ, VP, VP, SZ, VP, VP, SZ, VP, VP, SZ, VP]),
    "ts_hip_gemm_workspace_floats": (SZ, [SZ, SZ, SZ]),
    "ts_hip_gemm_batched": (_c.c_int, [_c.c_int, _c.c_int, SZ, SZ, SZ, VP, SZ, VP, SZ, VP, SZ, SZ,
                                       _c.POINTER(SZ), _c.POINTER(SZ), _c.POINTER(SZ), SZ, VP]),
    "ts_hip_gemv_workspace_floats": (SZ, [_c.c_int, SZ, SZ]),
    "ts_hip_gemv": (_c.c_int, [_c.c_int, SZ, SZ, VP, SZ, VP, VP, VP, SZ, VP]),
    "ts_hip_dot": (_c.c_int, [VP, VP, SZ, VP, VP, SZ, VP]),
    "ts_hip_outer": (_c.c_int, [VP, SZ, VP, SZ, VP, VP]),
    "ts_hip_adam_step": (_c.c_int, [VP, VP, VP, VP, VP, SZ, _c.c_float, _c.c_float, _c.c_float,
                                    _c.c_float, _c.c_float, _c.c_uint64, SZ, _c.c_int, VP]),
    "ts_hip_adam_step_multi": (_c.c_int, [VP, SZ, _c.c_float, _c.c_float, _c.c_float, _c.c_float,
                                          _c.c_float, _c.c_uint64, VP]),
    "ts_hip_adam_step_multi_table": (_c.c_int, [VP, SZ, _c.c_float, _c.c_float, _c.c_float, _c.c_float,
                                                _c.c_float, VP, VP, VP]),
    "ts_hip_adam_step_multi_ticket": (_c.c_int, [VP, SZ, _c.c_float, _c.c_float, _c.c_float, _c.c_float,
                                                 _c.c_float, VP, VP, VP]),
    "ts_hip_adam_multi_waves": (SZ, [VP, SZ]),
    "ts_hip_adam_bias_corrections": (_c.c_int, [_c.c_float, _c.c_float, _c.c_uint64, SZ, VP]),
    "ts_hip_slot_advance": (_c.c_int, [VP, VP]),
    "ts_hip_module_load_data": (_c.c_int, [VP, _c.POINTER(VP)]),
    "ts_hip_module_unload": (_c.c_int, [VP]),
    "ts_hip_module_get_function": (_c.c_int, [VP, _c.c_char_p, _c.POINTER(VP)]),
    "ts_hip_module_launch": (_c.c_int, [VP, _c.c_uint, _c.c_uint, _c.c_uint, _c.c_uint, _c.c_uint, _c.c_uint,
                                        _c.c_uint, VP, _c.POINTER(VP)]),
    "ts_hip_stream_begin_capture": (_c.c_int, [VP]),
    "ts_hip_stream_end_capture": (_c.c_int, [VP, _c.POINTER(VP)]),
    "ts_hip_stream_is_capturing": (_c.c_int, [VP, _c.POINTER(_c.c_int)]),
    "ts_hip_graph_launch": (_c.c_int, [VP, VP]),
    "ts_hip_graph_destroy": (_c.c_int, [VP]),
}


class AdamParam(ctypes.Structure):
    """struct ts_hip_adam_param of include/ts_hip.h"""
    _fields_ = [("p", VP), ("g", VP), ("m", VP), ("v", VP), ("v_hat_max", VP), ("n", SZ),
                ("amsgrad_first", _c.c_int)]

TP = VP  # opaque ts_tensor* / ts_adam*

# name -> (restype, argtypes); every symbol declared in include/ts_gradtrack.h
GRADTRACK_SIGNATURES = {
    "ts_last_error": (_c.c_char_p, []),
    "ts_tensor_new": (TP, [_c.POINTER(SZ), SZ]),
    "ts_tensor_zeros": (TP, [_c.POINTER(SZ), SZ]),
    "ts_tensor_ones": (TP, [_c.POINTER(SZ), SZ]),
    "ts_tensor_from_slice": (TP, [F, SZ, _c.POINTER(SZ), SZ]),
    "ts_tensor_randn": (TP, [_c.POINTER(SZ), SZ, _c.c_uint64, _c.c_int]),
    "ts_tensor_fill_randn": (_c.c_int, [TP, _c.c_uint64, _c.c_int]),
    "ts_tensor_clone": (TP, [TP]),
    "ts_tensor_free": (None, [TP]),
    "ts_tensor_id": (_c.c_uint64, [TP]),
    "ts_tensor_rank": (SZ, [TP]),
    "ts_tensor_dims": (SZ, [TP, _c.POINTER(SZ), SZ]),
    "ts_tensor_size": (SZ, [TP]),
    "ts_tensor_device_ptr": (VP, [TP]),
    "ts_tensor_with_requires_grad": (_c.c_int, [TP]),
    "ts_tensor_set_requires_grad": (_c.c_int, [TP, _c.c_int]),
    "ts_tensor_requires_grad": (_c.c_int, [TP]),
    "ts_tensor_add_tensor": (TP, [TP, TP]),
    "ts_tensor_sub_tensor": (TP, [TP, TP]),
    "ts_tensor_mul_tensor": (TP, [TP, TP]),
    "ts_tensor_div_tensor": (TP, [TP, TP]),
    "ts_tensor_add_scalar": (TP, [TP, _c.c_float]),
    "ts_tensor_sub_scalar": (TP, [TP, _c.c_float]),
    "ts_tensor_mul_scalar": (TP, [TP, _c.c_float]),
    "ts_tensor_div_scalar": (TP, [TP, _c.c_float]),
    "ts_tensor_relu": (TP, [TP]),
    "ts_tensor_pow_scalar": (TP, [TP, _c.c_float]),
    "ts_tensor_matmul": (TP, [TP, TP]),
    "ts_tensor_exp": (TP, [TP]),
    "ts_tensor_log": (TP, [TP]),
    "ts_tensor_sqrt": (TP, [TP]),
    "ts_tensor_tanh": (TP, [TP]),
    "ts_tensor_sigmoid": (TP, [TP]),
    "ts_tensor_leaky_relu": (TP, [TP, _c.c_float]),
    "ts_tensor_softmax": (TP, [TP, SZ]),
    "ts_tensor_sum_dims": (TP, [TP, _c.POINTER(SZ), SZ, _c.c_int]),
    "ts_tensor_mean_dims": (TP, [TP, _c.POINTER(SZ), SZ, _c.c_int]),
    "ts_tensor_transpose": (TP, [TP, SZ, SZ]),
    "ts_tensor_t": (TP, [TP]),
    "ts_tensor_contiguous": (TP, [TP]),
    "ts_tensor_is_contiguous": (_c.c_int, [TP]),
    "ts_tensor_fill": (_c.c_int, [TP, _c.c_float]),
    "ts_tensor_sum": (TP, [TP]),
    "ts_tensor_mean": (TP, [TP]),
    "ts_tensor_backward": (_c.c_int, [TP, TP]),
    "ts_tensor_grad": (TP, [TP]),
    "ts_tensor_grad_by_value": (TP, [TP]),
    "ts_tensor_set_grad": (_c.c_int, [TP, TP]),
    "ts_tensor_zero_grad": (_c.c_int, [TP]),
    "ts_tensor_data": (_c.c_int, [TP, F, SZ]),
    "ts_tensor_value": (_c.c_int, [TP, F]),
    "ts_clear_gradients": (None, []),
    "ts_no_grad_push": (None, []),
    "ts_no_grad_pop": (None, []),
    "ts_is_grad_enabled": (_c.c_int, []),
    "ts_set_grad_enabled": (None, [_c.c_int]),
    "ts_adam_new": (TP, []),
    "ts_adam_with_config": (TP, [_c.c_float, _c.c_float, _c.c_float, _c.c_float, _c.c_float, _c.c_int]),
    "ts_adam_with_learning_rate": (TP, [_c.c_float]),
    "ts_adam_free": (None, [TP]),
    "ts_adam_add_parameter": (_c.c_int, [TP, TP]),
    "ts_adam_step": (_c.c_int, [TP, _c.POINTER(TP), SZ]),
    "ts_adam_zero_grad": (_c.c_int, [TP, _c.POINTER(TP), SZ]),
    "ts_adam_learning_rate": (_c.c_float, [TP]),
    "ts_adam_set_learning_rate": (None, [TP, _c.c_float]),
    "ts_adam_step_count": (_c.c_uint64, [TP]),
    "ts_adam_state": (_c.c_int, [TP, TP, _c.c_int, F, SZ]),
    "ts_buffer_free": (None, [VP]),
    "ts_tensor_to_binary": (_c.c_int, [TP, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_tensor_from_binary": (TP, [VP, SZ]),
    "ts_tensor_to_json": (_c.c_int, [TP, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_tensor_from_json": (TP, [_c.c_char_p, SZ]),
    "ts_tensor_save_binary": (_c.c_int, [TP, _c.c_char_p]),
    "ts_tensor_save_json": (_c.c_int, [TP, _c.c_char_p]),
    "ts_tensor_load_binary": (TP, [_c.c_char_p]),
    "ts_tensor_load_json": (TP, [_c.c_char_p]),
    "ts_adam_to_binary": (_c.c_int, [TP, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_adam_from_binary": (TP, [VP, SZ]),
    "ts_adam_to_json": (_c.c_int, [TP, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_adam_from_json": (TP, [_c.c_char_p, SZ]),
    "ts_adam_save_binary": (_c.c_int, [TP, _c.c_char_p]),
    "ts_adam_save_json": (_c.c_int, [TP, _c.c_char_p]),
    "ts_adam_load_binary": (TP, [_c.c_char_p]),
    "ts_adam_load_json": (TP, [_c.c_char_p]),
    "ts_adam_relink_parameters": (_c.c_int, [TP, _c.POINTER(TP), SZ]),
    "ts_adam_saved_parameter_count": (SZ, [TP]),
    "ts_adam_parameter_step": (_c.c_uint64, [TP, TP]),
    "ts_adam_config": (_c.c_int, [TP, F, _c.POINTER(_c.c_int)]),
    "ts_adam_config_to_binary": (_c.c_int, [F, _c.c_int, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_adam_config_from_binary": (_c.c_int, [VP, SZ, F, _c.POINTER(_c.c_int)]),
    "ts_adam_config_to_json": (_c.c_int, [F, _c.c_int, _c.POINTER(VP), _c.POINTER(SZ)]),
    "ts_adam_config_from_json": (_c.c_int, [_c.c_char_p, SZ, F, _c.POINTER(_c.c_int)]),
    "ts_synchronize": (_c.c_int, []),
    "ts_fusion_enable": (None, [_c.c_int]),
    "ts_fusion_enabled": (_c.c_int, []),
    "ts_step_graph_begin": (_c.c_int, []),
    "ts_step_graph_end": (TP, []),
    "ts_step_graph_abort": (None, []),
    "ts_step_graph_recording": (_c.c_int, []),
    "ts_step_graph_replay": (_c.c_int, [TP, SZ]),
    "ts_step_graph_free": (None, [TP]),
    "ts_stream": (VP, []),
    "ts_pool_live_bytes": (SZ, []),
    "ts_pool_cached_bytes": (SZ, []),
    "ts_pool_empty_cache": (None, []),
    "ts_profile_classes": (None, [_c.c_uint]),
    "ts_profile_enable": (None, [_c.c_int]),
    "ts_profile_reset": (None, []),
    "ts_profile_read": (_c.c_int, [_c.c_int, _c.POINTER(_c.c_double), _c.POINTER(_c.c_double),
                                   _c.POINTER(_c.c_uint64)]),
}


def _bind(lib: ctypes.CDLL, sigs: dict) -> ctypes.CDLL:
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)  # AttributeError if the library lacks a declared symbol
        fn.restype = res
        fn.argtypes = args
    return lib


hip = _bind(_load("libts_hip.so"), HIP_SIGNATURES)
gradtrack = _bind(_load("libts_gradtrack.so"), GRADTRACK_SIGNATURES)


def hip_check(status: int, what: str = "ts_hip") -> None:
    if status != 0:
        msg = hip.ts_hip_error_string(status).decode()
        raise TsError(f"{what}: {msg} (status {status})")


def last_error() -> str:
    return gradtrack.ts_last_error().decode()
