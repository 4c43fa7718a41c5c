"""ctypes binding of libsimdyolo_hip.so (the C ABI in include/simdyolo_hip.h).

The library is built in-tree by ``simdyolo_amd.build`` (``__graft_entry__.build()``).
There is no fallback: if the shared object is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libsimdyolo_hip.so")

SY_OK, SY_EINVAL, SY_EUNSUPPORTED, SY_EDEVICE, SY_ENOMEM, SY_ESTATE = range(6)
LAYOUT_NHWC, LAYOUT_NCHW = 0, 1
CONV_AUTO, CONV_IGEMM, CONV_WINOGRAD, CONV_DIRECT, CONV_WINOGRAD3, CONV_DEPTHWISE, CONV_WINOGRAD2 = range(7)
ARCH_YOLOV8, ARCH_YOLO11, ARCH_YOLO26 = 0, 1, 2

# Every exported symbol declared in include/simdyolo_hip.h.
EXPORTS = (
    "sy_create", "sy_destroy", "sy_name", "sy_last_error", "sy_device_count", "sy_version",
    "sy_frame_begin", "sy_frame_end", "sy_flush", "sy_frame_alloc", "sy_upload_nchw", "sy_download_nchw",
    "sy_malloc", "sy_free", "sy_memcpy",
    "sy_conv_create", "sy_conv_transpose2x2_create", "sy_conv_set_algo", "sy_conv_get_algo", "sy_conv_run",
    "sy_conv_run_upsampled", "sy_conv_out_size", "sy_tune_save", "sy_tune_load",
    "sy_add", "sy_resize_nearest", "sy_maxpool", "sy_sppf_pool", "sy_copy", "sy_detect_decode", "sy_e2e_topk",
    "sy_e2e_topk_noalloc",
    "sy_mask_decode", "sy_attention", "sy_compute", "sy_matmul",
    "sy_graph_begin", "sy_graph_end", "sy_graph_launch", "sy_graph_destroy",
    "sy_timer_start", "sy_timer_stop", "sy_profile_enable", "sy_profile_read",
    "sy_model_layout", "sy_model_create", "sy_model_destroy", "sy_model_output_shape", "sy_model_predict_raw",
    "sy_model_buffers", "sy_model_run", "sy_model_set_graph", "sy_model_set_branch_level",
    "sy_model_branch_level", "sy_model_memory", "sy_model_plan_memory", "sy_model_proto", "sy_model_head",
    "sy_model_predict_seg",
    "sy_decode_detections", "sy_letterbox_rgb", "sy_letterbox_device", "sy_nms_candidates",
    "sy_decode_detections_device", "sy_fold_bn",
)


class SyError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class Tensor(ctypes.Structure):
    """sy_tensor: NHWC view (or dense NCHW when layout == 1)."""
    _fields_ = [("data", ctypes.c_void_p), ("n", ctypes.c_int32), ("c", ctypes.c_int32),
                ("h", ctypes.c_int32), ("w", ctypes.c_int32), ("ldc", ctypes.c_int32),
                ("layout", ctypes.c_int32)]

    def slice(self, c0: int, count: int) -> "Tensor":
        assert self.layout == LAYOUT_NHWC and 0 <= c0 and c0 + count <= self.c
        return Tensor(self.data + 4 * c0, self.n, count, self.h, self.w, self.ldc, self.layout)

    @property
    def shape(self):
        return (self.n, self.c, self.h, self.w)


class ModelConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int32), ("depth", ctypes.c_float), ("width", ctypes.c_float),
                ("max_channels", ctypes.c_int32), ("nc", ctypes.c_int32), ("reg_max", ctypes.c_int32),
                ("bn_eps", ctypes.c_float), ("nm", ctypes.c_int32), ("npr", ctypes.c_int32)]


class LetterboxT(ctypes.Structure):
    _fields_ = [("source_width", ctypes.c_int32), ("source_height", ctypes.c_int32),
                ("target_width", ctypes.c_int32), ("target_height", ctypes.c_int32),
                ("scale_x", ctypes.c_float), ("scale_y", ctypes.c_float),
                ("pad_x", ctypes.c_int32), ("pad_y", ctypes.c_int32)]


class DetectionT(ctypes.Structure):
    _fields_ = [("class_id", ctypes.c_int32), ("confidence", ctypes.c_float), ("x", ctypes.c_float),
                ("y", ctypes.c_float), ("width", ctypes.c_float), ("height", ctypes.c_float),
                ("anchor", ctypes.c_int32)]


class MaskInfo(ctypes.Structure):
    _fields_ = [("left", ctypes.c_int32), ("top", ctypes.c_int32), ("width", ctypes.c_int32),
                ("height", ctypes.c_int32), ("offset", ctypes.c_int64)]


class DecodeOptions(ctypes.Structure):
    _fields_ = [("confidence", ctypes.c_float), ("iou", ctypes.c_float), ("max_detections", ctypes.c_int32),
                ("max_candidates", ctypes.c_int32), ("class_count", ctypes.c_int32),
                ("agnostic", ctypes.c_int32), ("layout", ctypes.c_int32)]


_lib = None
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_fp = ctypes.POINTER(ctypes.c_float)
_tp = ctypes.POINTER(Tensor)
_u64p = ctypes.POINTER(ctypes.c_uint64)

_SIGS = {
    "sy_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "sy_destroy": (None, [_vp]),
    "sy_name": (ctypes.c_char_p, [_vp]),
    "sy_last_error": (ctypes.c_char_p, []),
    "sy_device_count": (_i, [ctypes.POINTER(_i)]),
    "sy_version": (ctypes.c_char_p, []),
    "sy_frame_begin": (_i, [_vp, ctypes.POINTER(ctypes.c_int64)]),
    "sy_frame_end": (_i, [_vp]),
    "sy_flush": (_i, [_vp]),
    "sy_frame_alloc": (_i, [_vp, _i, _i, _i, _i, _tp]),
    "sy_upload_nchw": (_i, [_vp, _fp, _tp]),
    "sy_download_nchw": (_i, [_vp, _tp, _fp]),
    "sy_malloc": (_i, [_vp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "sy_free": (_i, [_vp, _vp]),
    "sy_memcpy": (_i, [_vp, _vp, _vp, ctypes.c_size_t, _i]),
    "sy_conv_create": (_i, [_vp, _fp, _fp] + [_i] * 14 + [_u64p]),
    "sy_conv_transpose2x2_create": (_i, [_vp, _fp, _fp, _i, _i, _u64p]),
    "sy_conv_set_algo": (_i, [_vp, ctypes.c_uint64, _i]),
    "sy_conv_get_algo": (_i, [_vp, ctypes.c_uint64, ctypes.POINTER(_i)]),
    "sy_conv_run": (_i, [_vp, ctypes.c_uint64, _tp, _tp, _tp]),
    "sy_conv_run_upsampled": (_i, [_vp, ctypes.c_uint64, _tp, _tp, _tp, _tp]),
    "sy_conv_out_size": (_i, [_vp, ctypes.c_uint64, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "sy_tune_save": (_i, [_vp, ctypes.c_char_p]),
    "sy_tune_load": (_i, [_vp, ctypes.c_char_p]),
    "sy_add": (_i, [_vp, _tp, _tp, _tp]),
    "sy_resize_nearest": (_i, [_vp, _tp, _tp]),
    "sy_maxpool": (_i, [_vp, _tp, _tp] + [_i] * 9),
    "sy_sppf_pool": (_i, [_vp, _tp, _tp, _tp, _tp]),
    "sy_copy": (_i, [_vp, _tp, _tp]),
    "sy_detect_decode": (_i, [_vp, _tp, _fp, _i, _i, _i, _i, _vp, _i]),
    "sy_e2e_topk": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "sy_e2e_topk_noalloc": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "sy_mask_decode": (_i, [_vp, _tp, _vp, _i, _i, ctypes.POINTER(DetectionT), ctypes.POINTER(LetterboxT), _vp,
                            ctypes.c_size_t, ctypes.POINTER(MaskInfo)]),
    "sy_attention": (_i, [_vp, _tp, _i, _i, _i, _f, _tp, _tp]),
    "sy_compute": (_i, [_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_uint32),
                        ctypes.c_int64, _vp, ctypes.c_size_t]),
    "sy_matmul": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, ctypes.POINTER(ctypes.c_int32),
                       ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64), ctypes.c_size_t,
                       ctypes.c_size_t, ctypes.c_size_t]),
    "sy_graph_begin": (_i, [_vp]),
    "sy_graph_end": (_i, [_vp, _u64p]),
    "sy_graph_launch": (_i, [_vp, ctypes.c_uint64]),
    "sy_graph_destroy": (_i, [_vp, ctypes.c_uint64]),
    "sy_timer_start": (_i, [_vp]),
    "sy_timer_stop": (_i, [_vp, _fp]),
    "sy_profile_enable": (_i, [_vp, _i]),
    "sy_profile_read": (_i, [_vp, ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_i), _fp,
                             ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), _i,
                             ctypes.POINTER(_i)]),
    "sy_model_layout": (_i, [ctypes.POINTER(ModelConfig), ctypes.POINTER(ctypes.c_int32), _i, ctypes.POINTER(_i)]),
    "sy_model_create": (_i, [_vp, ctypes.POINTER(ModelConfig), _fp, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "sy_model_destroy": (None, [_vp]),
    "sy_model_output_shape": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "sy_model_predict_raw": (_i, [_vp, _fp, _i, _i, _i, _fp]),
    "sy_model_buffers": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
    "sy_model_run": (_i, [_vp, _i, _i, _i]),
    "sy_model_set_graph": (_i, [_vp, _i]),
    "sy_model_set_branch_level": (_i, [_vp, _i]),
    "sy_model_branch_level": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_i)]),
    "sy_model_memory": (_i, [_vp, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "sy_model_plan_memory": (_i, [_vp, _i, _i, _i] + [ctypes.POINTER(ctypes.c_size_t)] * 3),
    "sy_model_head": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "sy_model_proto": (_i, [_vp, _i, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_i), ctypes.POINTER(_i),
                            ctypes.POINTER(_i)]),
    "sy_model_predict_seg": (_i, [_vp, _fp, _i, _i, _i, _fp, _fp]),
    "sy_decode_detections": (_i, [_fp, _i, _i, ctypes.POINTER(DecodeOptions), ctypes.POINTER(LetterboxT),
                                  ctypes.POINTER(DetectionT), _i, ctypes.POINTER(_i)]),
    "sy_letterbox_rgb": (_i, [ctypes.POINTER(ctypes.c_uint8), _i, _i, _i, _i, _i, _i, _fp,
                              ctypes.POINTER(LetterboxT)]),
    "sy_letterbox_device": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _vp, ctypes.POINTER(LetterboxT)]),
    "sy_nms_candidates": (_i, [_vp, _vp, _i, _i, _i, ctypes.POINTER(DecodeOptions), _vp, _vp]),
    "sy_decode_detections_device": (_i, [_vp, _vp, _i, _i, _i, ctypes.POINTER(DecodeOptions),
                                         ctypes.POINTER(LetterboxT), ctypes.POINTER(DetectionT), _i,
                                         ctypes.POINTER(_i)]),
    "sy_fold_bn": (None, [_fp, _i, _i, _fp, _fp, _fp, _fp, _fp, _f, _fp, _fp]),
}


def lib() -> ctypes.CDLL:
    """Load the in-tree library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"libsimdyolo_hip.so not built at {LIB_PATH}; run __graft_entry__.build()")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int) -> None:
    if rc != SY_OK:
        raise SyError(rc, lib().sy_last_error().decode(errors="replace"))


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)
