"""ctypes binding of libsplathip (include/splathip.h, include/splathip_kernels.h).

The host-side mirror of the reference's entry points:
  Da3.load(path, variant, dtype, strategy)  ~ depthanything3-rs/src/weights.rs:26-48 load_model
  Da3.forward_raw(images)                   ~ depthanything3-rs/src/model.rs:101-123 forward_raw
  MapAnything.load(path, spec, dtype)       ~ mapanything-rs/src/model.rs:69-81 MapAnything::new
  MapAnything.forward(images)               ~ mapanything-rs/src/model.rs:86-144 forward
Errors raise SplatError carrying the library's status code and message (the reference's
Result errors / panics). The library is required: importing this module fails loudly when
libsplathip.so is missing.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

from . import specs

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libsplathip.so")

OK, BAD_ARGUMENT, BAD_SHAPE, MISSING_KEY, SHAPE_MISMATCH, HIP_ERROR, NONFINITE, IO_ERROR, NOT_LOADED = range(9)
F32, BF16, F16 = 0, 1, 2
DTYPES = {"f32": F32, "fp32": F32, "bf16": BF16, "f16": F16}
STAGE_BLOCK, STAGE_DENSE_HEAD, STAGE_CAMERA_HEAD = 0, 1, 2
FILTER_TRIANGLE, FILTER_CATMULLROM, FILTER_LANCZOS3 = 1, 2, 3   # image 0.25.10 imageops::FilterType


class SplatError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class MaSpecC(C.Structure):
    _fields_ = [("enc_dim", C.c_int), ("enc_heads", C.c_int), ("enc_depth", C.c_int), ("enc_ffn", C.c_int),
                ("enc_hidden", C.c_int), ("info_dim", C.c_int), ("info_heads", C.c_int), ("info_depth", C.c_int),
                ("info_ffn", C.c_int), ("info_hidden", C.c_int), ("hooks", C.c_int * 3), ("dpt_dims", C.c_int * 4),
                ("dpt_features", C.c_int), ("pose_dim", C.c_int), ("scale_dim", C.c_int)]

    @classmethod
    def from_spec(cls, s: specs.MaSpec) -> "MaSpecC":
        return cls(s.enc_dim, s.enc_heads, s.enc_depth, s.enc_ffn, s.enc_hidden, s.info_dim, s.info_heads,
                   s.info_depth, s.info_ffn, s.info_hidden, (C.c_int * 3)(*s.hooks), (C.c_int * 4)(*s.dpt_dims),
                   s.dpt_features, s.pose_dim, s.scale_dim)


class Da3OutC(C.Structure):
    _fields_ = [("depth", C.c_void_p), ("depth_conf", C.c_void_p), ("ray_logits", C.c_void_p),
                ("pose_encoding", C.c_void_p), ("camera_tokens", C.c_void_p), ("reference_view", C.c_int32)]


class MaOutC(C.Structure):
    _fields_ = [("raw", C.c_void_p), ("quaternion", C.c_void_p), ("translation", C.c_void_p), ("scale", C.c_void_p),
                ("points", C.c_void_p), ("conf", C.c_void_p), ("mask", C.c_void_p)]


class ReconOutC(C.Structure):
    _fields_ = [("points", C.c_void_p), ("conf", C.c_void_p), ("depth", C.c_void_p), ("rotation", C.c_void_p),
                ("translation", C.c_void_p), ("focal", C.c_void_p), ("principal_point", C.c_void_p),
                ("reference_view", C.c_int32)]


class KernelStatC(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_int), ("ms", C.c_double), ("flops", C.c_double),
                ("bytes", C.c_double)]


PROGRESS_FN = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)
TAP_FN = C.CFUNCTYPE(None, C.c_int, C.POINTER(C.c_float), C.c_int, C.c_int, C.c_void_p)
BRANCH_TAP_FN = C.CFUNCTYPE(None, C.c_int, C.c_int, C.POINTER(C.c_float), C.c_int, C.c_int, C.c_void_p)

# Every symbol the two public headers declare, with its ctypes signature.
SIGNATURES = {
    "splat_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "splat_destroy": (None, [C.c_void_p]),
    "splat_last_error": (C.c_char_p, [C.c_void_p]),
    "splat_stream": (C.c_void_p, [C.c_void_p]),
    "splat_synchronize": (C.c_int, [C.c_void_p]),
    "splat_set_graphs": (C.c_int, [C.c_void_p, C.c_int]),
    "splat_set_debug_taps": (C.c_int, [C.c_void_p, TAP_FN, C.c_void_p]),
    "splat_set_branch_taps": (C.c_int, [C.c_void_p, BRANCH_TAP_FN, C.c_void_p]),
    "splat_load_da3": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int, C.c_int, C.c_int]),
    "splat_load_da3_bytes": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int]),
    "splat_da3_forward_raw": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, PROGRESS_FN, C.c_void_p,
                                        C.POINTER(Da3OutC)]),
    "splat_da3_forward_raw_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(Da3OutC),
                                               C.c_void_p]),
    "splat_load_mapanything": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(MaSpecC), C.c_int]),
    "splat_load_mapanything_bytes": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(MaSpecC), C.c_int]),
    "splat_ma_reference_spec": (None, [C.POINTER(MaSpecC)]),
    "splat_ma_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.POINTER(MaOutC)]),
    "splat_ma_forward_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                          C.POINTER(MaOutC)]),
    "splat_ma_encode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "splat_to_model_input": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "splat_da3_reconstruct": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                        C.POINTER(ReconOutC)]),
    "splat_ma_reconstruct": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                       C.POINTER(ReconOutC)]),
    "splat_ma_encode_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "splat_kernel_gemm": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int,
                                    C.c_void_p, C.c_int, C.c_void_p, C.c_int]),
    "splat_kernel_gemm_ln": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                       C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_float, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int]),
    "splat_kernel_ln_stats": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                        C.c_void_p]),
    "splat_kernel_attention": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "splat_kernel_attention_noalloc": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                                 C.c_int]),
    "splat_profile_begin": (C.c_int, [C.c_void_p]),
    "splat_profile_end": (C.c_int, [C.c_void_p, C.POINTER(KernelStatC), C.c_int, C.POINTER(C.c_int)]),
    "splat_kernel_conv2d": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                      C.c_void_p]),
    "splat_kernel_conv_transpose2d": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                                C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "splat_kernel_resize_bilinear": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                               C.c_void_p, C.c_int, C.c_int]),
    "splat_kernel_reconstruct": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int] + [C.c_void_p] * 11),
    "splat_resize_rgba8": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "splat_da3_input_size": (C.c_int, [C.c_int, C.c_int] + [C.POINTER(C.c_int)] * 4),
    "splat_ma_input_size": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "splat_da3_model_inputs": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "splat_ma_model_inputs": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library (RTLD_LOCAL), with every declared symbol typed."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `make -C splatting-rs_amd` "
                              "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data) if a is not None else C.c_void_p(0)


class Context:
    """One HIP stream + weights + activation arena on a device (splat_create)."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        h = C.c_void_p()
        rc = self._lib.splat_create(device, C.byref(h))
        if rc != OK:
            raise SplatError(rc, self._lib.splat_last_error(None).decode())
        self.handle = h
        self._callbacks = []

    def close(self):
        if self.handle:
            self._lib.splat_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc: int):
        if rc != OK:
            raise SplatError(rc, self._lib.splat_last_error(self.handle).decode())

    @property
    def stream(self) -> int:
        return self._lib.splat_stream(self.handle)

    def synchronize(self):
        self.check(self._lib.splat_synchronize(self.handle))

    def set_graphs(self, enable: bool):
        self.check(self._lib.splat_set_graphs(self.handle, int(enable)))

    def set_debug_taps(self, fn):
        """fn(block, ndarray [rows, dim]) per block, or None."""
        if fn is None:
            self.check(self._lib.splat_set_debug_taps(self.handle, TAP_FN(), None))
            return
        def tap(block, ptr, rows, dim, user):
            fn(block, np.ctypeslib.as_array(ptr, shape=(rows, dim)).copy())
        cb = TAP_FN(tap)
        self._callbacks.append(cb)
        self.check(self._lib.splat_set_debug_taps(self.handle, cb, None))

    def set_branch_taps(self, fn):
        """fn(block, branch, ndarray [rows, dim]) per block and branch (0 attention, 1
        feed-forward; the branch output before its LayerScale), or None."""
        if fn is None:
            self.check(self._lib.splat_set_branch_taps(self.handle, BRANCH_TAP_FN(), None))
            return
        def tap(block, branch, ptr, rows, dim, user):
            fn(block, branch, np.ctypeslib.as_array(ptr, shape=(rows, dim)).copy())
        cb = BRANCH_TAP_FN(tap)
        self._callbacks.append(cb)
        self.check(self._lib.splat_set_branch_taps(self.handle, cb, None))

    # --- Depth Anything 3 -------------------------------------------------------------------
    def load_da3(self, path: str, variant: str = "small", dtype: str = "f32", strategy: int = specs.REF_SADDLE):
        self.check(self._lib.splat_load_da3(self.handle, path.encode(), specs.DA3_VARIANT_INDEX[variant],
                                            DTYPES[dtype], strategy))
        self.da3_spec = specs.DA3_VARIANTS[variant]

    def load_da3_bytes(self, data: bytes, variant: str = "small", dtype: str = "f32", strategy: int = specs.REF_SADDLE):
        buf = np.frombuffer(data, np.uint8)
        self.check(self._lib.splat_load_da3_bytes(self.handle, _ptr(buf), buf.size, specs.DA3_VARIANT_INDEX[variant],
                                                  DTYPES[dtype], strategy))
        self.da3_spec = specs.DA3_VARIANTS[variant]

    def da3_forward_raw(self, images: np.ndarray, progress=None, rays: bool = True, camera_tokens: bool = True,
                        allow_nonfinite: bool = False) -> dict:
        x = np.ascontiguousarray(images, np.float32)
        V, _, H, W = x.shape
        R, Cc = H // 14, W // 14
        d = self.da3_spec.dim
        out = {
            "depth": np.empty((V, H, W), np.float32),
            "depth_conf": np.empty((V, H, W), np.float32),
            "ray_logits": np.empty((V, 7, 8 * R, 8 * Cc), np.float32) if rays else None,
            "pose_encoding": np.empty((V, 9), np.float32),
            "camera_tokens": np.empty((V, 2 * d), np.float32) if camera_tokens else None,
        }
        o = Da3OutC(*[_ptr(out[k]) for k in ("depth", "depth_conf", "ray_logits", "pose_encoding", "camera_tokens")], 0)
        cb = PROGRESS_FN(lambda s, b, u: progress(s, b)) if progress else PROGRESS_FN()
        rc = self._lib.splat_da3_forward_raw(self.handle, _ptr(x), V, H, W, cb, None, C.byref(o))
        if not (allow_nonfinite and rc == NONFINITE):
            self.check(rc)
        out["reference_view"] = int(o.reference_view)
        return out

    def da3_forward_raw_device(self, images_ptr: int, V: int, H: int, W: int, outs: dict, ref_ptr: int = 0):
        o = Da3OutC(*[C.c_void_p(outs.get(k) or 0) for k in
                      ("depth", "depth_conf", "ray_logits", "pose_encoding", "camera_tokens")], 0)
        self.check(self._lib.splat_da3_forward_raw_device(self.handle, C.c_void_p(images_ptr), V, H, W, C.byref(o),
                                                          C.c_void_p(ref_ptr)))

    # --- MapAnything ------------------------------------------------------------------------
    def load_mapanything(self, path: str, spec: Optional[specs.MaSpec] = None, dtype: str = "bf16"):
        cs = MaSpecC.from_spec(spec) if spec is not None else None
        self.check(self._lib.splat_load_mapanything(self.handle, path.encode(), C.byref(cs) if cs else None,
                                                    DTYPES[dtype]))
        self.ma_spec = spec or specs.MA_SPECS["reference"]

    def load_mapanything_bytes(self, data: bytes, spec: Optional[specs.MaSpec] = None, dtype: str = "bf16"):
        """A safetensors checkpoint held in memory (the wasm worker's fetched bytes)."""
        buf = np.frombuffer(data, np.uint8)
        cs = MaSpecC.from_spec(spec) if spec is not None else None
        self.check(self._lib.splat_load_mapanything_bytes(self.handle, _ptr(buf), buf.size,
                                                          C.byref(cs) if cs else None, DTYPES[dtype]))
        self.ma_spec = spec or specs.MA_SPECS["reference"]

    @staticmethod
    def _cameras(intrinsics, V: int):
        """None, or one entry per view: None (unknown camera) or (fx, fy, cx, cy)."""
        if intrinsics is None:
            return None
        assert len(intrinsics) == V, "one intrinsics entry per view"
        k = np.zeros((V, 4), np.float64)
        for v, e in enumerate(intrinsics):
            k[v] = e if e is not None else (np.nan, np.nan, np.nan, np.nan)
        return k

    def ma_forward(self, images: np.ndarray, raw: bool = True, dense: bool = True, intrinsics=None) -> dict:
        x = np.ascontiguousarray(images, np.float32)
        V, _, H, W = x.shape
        out = {
            "raw": np.empty((V, 6, H, W), np.float32) if raw else None,
            "quaternion": np.empty((V, 4), np.float32),
            "translation": np.empty((V, 3), np.float32),
            "scale": np.empty((1,), np.float32),
            "points": np.empty((V, H, W, 3), np.float32) if dense else None,
            "conf": np.empty((V, H, W), np.float32) if dense else None,
            "mask": np.empty((V, H, W), np.uint8) if dense else None,
        }
        o = MaOutC(*[_ptr(out[k]) for k in ("raw", "quaternion", "translation", "scale", "points", "conf", "mask")])
        k = self._cameras(intrinsics, V)
        self.check(self._lib.splat_ma_forward(self.handle, _ptr(x), V, H, W, _ptr(k) if k is not None else None,
                                              C.byref(o)))
        return out

    def ma_forward_device(self, images_ptr: int, V: int, H: int, W: int, outs: dict, intrinsics=None):
        o = MaOutC(*[C.c_void_p(outs.get(k) or 0) for k in
                     ("raw", "quaternion", "translation", "scale", "points", "conf", "mask")])
        k = self._cameras(intrinsics, V)
        self.check(self._lib.splat_ma_forward_device(self.handle, C.c_void_p(images_ptr), V, H, W,
                                                     _ptr(k) if k is not None else None, C.byref(o)))

    @staticmethod
    def _recon_out(V: int, H: int, W: int):
        out = {"points": np.empty((V, H, W, 3), np.float32), "conf": np.empty((V, H, W), np.float32),
               "depth": np.empty((V, H, W), np.float32), "rotation": np.empty((V, 3, 3), np.float64),
               "translation": np.empty((V, 3), np.float64), "focal": np.empty((V, 2), np.float64),
               "principal_point": np.empty((V, 2), np.float64)}
        o = ReconOutC(*[_ptr(out[k]) for k in ("points", "conf", "depth", "rotation", "translation", "focal",
                                                "principal_point")], 0)
        return out, o

    def to_model_input_device(self, rgba: np.ndarray, images_ptr: int, foreground_ptr: int = 0):
        """RGBA u8 [V, H, W, 4] (host) -> normalised images and foreground in device memory."""
        x = np.ascontiguousarray(rgba, np.uint8)
        V, H, W, _ = x.shape
        self.check(self._lib.splat_to_model_input(self.handle, _ptr(x), V, H, W, C.c_void_p(images_ptr),
                                                  C.c_void_p(foreground_ptr or 0)))

    def resize_rgba8(self, rgba: np.ndarray, new_width: int, new_height: int, filter_type: int) -> np.ndarray:
        """image::imageops::resize of a host RGBA8 [h, w, 4] image, computed on the device."""
        x = np.ascontiguousarray(rgba, np.uint8)
        h, w, _ = x.shape
        out = np.empty((new_height, new_width, 4), np.uint8)
        self.check(self._lib.splat_resize_rgba8(self.handle, _ptr(x), w, h, _ptr(out), new_width, new_height,
                                                filter_type))
        return out

    def _model_inputs(self, fn, images, images_ptr: int, foreground_ptr: int):
        xs = [np.ascontiguousarray(im, np.uint8) for im in images]
        n = len(xs)
        ptrs = (C.c_void_p * n)(*[x.ctypes.data for x in xs])
        ws = np.array([x.shape[1] for x in xs], np.int32)
        hs = np.array([x.shape[0] for x in xs], np.int32)
        H, W = C.c_int(), C.c_int()
        self.check(fn(self.handle, n, ptrs, _ptr(ws), _ptr(hs), C.c_void_p(images_ptr), C.c_void_p(foreground_ptr or 0),
                      C.byref(H), C.byref(W)))
        return H.value, W.value

    def da3_model_inputs_device(self, images, images_ptr: int, foreground_ptr: int = 0):
        """depthanything3-rs/src/preprocess.rs:86-123 from decoded host RGBA8 images [h, w, 4] to the
        device model input (size from da3_model_input_size); returns (H, W)."""
        return self._model_inputs(self._lib.splat_da3_model_inputs, images, images_ptr, foreground_ptr)

    def ma_model_inputs_device(self, images, images_ptr: int, foreground_ptr: int = 0):
        """mapanything-rs/src/preprocess.rs:66-80 from decoded host RGBA8 images to the device
        model input (size from ma_input_size); returns (H, W)."""
        return self._model_inputs(self._lib.splat_ma_model_inputs, images, images_ptr, foreground_ptr)

    def da3_reconstruct(self, images: np.ndarray, foreground=None) -> dict:
        """depthanything3-rs/src/pipeline.rs:52-133 with the geometry on the device."""
        x = np.ascontiguousarray(images, np.float32)
        V, _, H, W = x.shape
        out, o = self._recon_out(V, H, W)
        fg = None if foreground is None else np.ascontiguousarray(foreground, np.uint8)
        self.check(self._lib.splat_da3_reconstruct(self.handle, _ptr(x), V, H, W, _ptr(fg) if fg is not None else None,
                                                   C.byref(o)))
        out["reference_view"] = int(o.reference_view)
        return out

    def ma_reconstruct(self, images: np.ndarray, intrinsics=None, foreground=None) -> dict:
        """mapanything-rs/src/pipeline.rs:41-104 with the geometry on the device."""
        x = np.ascontiguousarray(images, np.float32)
        V, _, H, W = x.shape
        out, o = self._recon_out(V, H, W)
        k = self._cameras(intrinsics, V)
        fg = None if foreground is None else np.ascontiguousarray(foreground, np.uint8)
        self.check(self._lib.splat_ma_reconstruct(self.handle, _ptr(x), V, H, W, _ptr(k) if k is not None else None,
                                                  _ptr(fg) if fg is not None else None, C.byref(o)))
        return out

    def ma_encode(self, images: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(images, np.float32)
        V, _, H, W = x.shape
        n = 1 + (H // 14) * (W // 14)
        tok = np.empty((V, n, self.ma_spec.enc_dim), np.float32)
        self.check(self._lib.splat_ma_encode(self.handle, _ptr(x), V, H, W, _ptr(tok)))
        return tok

    def ma_encode_device(self, images_ptr: int, V: int, H: int, W: int, tokens_ptr: int):
        self.check(self._lib.splat_ma_encode_device(self.handle, C.c_void_p(images_ptr), V, H, W, C.c_void_p(tokens_ptr)))

    # --- profiling ----------------------------------------------------------------------------
    def profile_begin(self):
        self.check(self._lib.splat_profile_begin(self.handle))

    def profile_end(self) -> list:
        """[{name, launches, ms, flops, bytes}], largest total time first."""
        stats = (KernelStatC * 64)()
        n = C.c_int()
        self.check(self._lib.splat_profile_end(self.handle, stats, 64, C.byref(n)))
        return [{"name": s.name.decode(), "launches": s.launches, "ms": s.ms, "flops": s.flops, "bytes": s.bytes}
                for s in stats[:n.value]]

    # --- kernels ------------------------------------------------------------------------------
    def kernel_gemm(self, dtype: int, A: int, M: int, K: int, W: int, N: int, ldw: int, bias: int, act: int,
                    out: int, out_f32: bool):
        self.check(self._lib.splat_kernel_gemm(self.handle, dtype, C.c_void_p(A), M, K, C.c_void_p(W), N, ldw,
                                               C.c_void_p(bias), act, C.c_void_p(out), int(out_f32)))

    def kernel_gemm_ln(self, dtype: int, A: int, M: int, K: int, W: int, N: int, ldw: int, bias: int, act: int,
                       out: int, out_f32: bool, ln_in: int = 0, c1: int = 0, eps: float = 1e-6, gamma: int = 0,
                       res: int = 0, ln_out: int = 0, copy: int = 0, group: int = 64):
        """splat_kernel_gemm_ln (device pointers as ints, 0 for NULL)."""
        v = lambda p: C.c_void_p(p or None)
        self.check(self._lib.splat_kernel_gemm_ln(self.handle, dtype, v(A), M, K, v(W), N, ldw, v(bias), act, v(ln_in),
                                                  v(c1), eps, v(gamma), v(res), v(ln_out), v(copy), group, v(out),
                                                  int(out_f32)))

    def kernel_ln_stats(self, x: int, rows: int, n: int, group: int, stats: int, dtype: int, copy: int = 0):
        self.check(self._lib.splat_kernel_ln_stats(self.handle, C.c_void_p(x), rows, n, group, C.c_void_p(stats),
                                                   dtype, C.c_void_p(copy or None)))

    def kernel_attention(self, dtype: int, qkv: int, out: int, S: int, L: int, heads: int):
        self.check(self._lib.splat_kernel_attention(self.handle, dtype, C.c_void_p(qkv), C.c_void_p(out), S, L, heads))

    def kernel_attention_noalloc(self, dtype: int, qkv: int, out: int, S: int, L: int, heads: int):
        self.check(self._lib.splat_kernel_attention_noalloc(self.handle, dtype, C.c_void_p(qkv), C.c_void_p(out), S, L,
                                                            heads))

    def kernel_conv2d(self, dtype, inp, V, H, W, Cin, w, Cout, ldw, ks, stride, bias, relu_in, act, res, out):
        self.check(self._lib.splat_kernel_conv2d(self.handle, dtype, C.c_void_p(inp), V, H, W, Cin, C.c_void_p(w), Cout,
                                                 ldw, ks, stride, C.c_void_p(bias), relu_in, act, C.c_void_p(res),
                                                 C.c_void_p(out)))

    def kernel_conv_transpose2d(self, dtype, inp, V, R, Cc, Cin, w, Cout, ldw, s, bias, out):
        self.check(self._lib.splat_kernel_conv_transpose2d(self.handle, dtype, C.c_void_p(inp), V, R, Cc, Cin,
                                                           C.c_void_p(w), Cout, ldw, s, C.c_void_p(bias),
                                                           C.c_void_p(out)))

    def kernel_resize_bilinear(self, dtype, inp, V, Hi, Wi, Cc, out, Ho, Wo):
        self.check(self._lib.splat_kernel_resize_bilinear(self.handle, dtype, C.c_void_p(inp), V, Hi, Wi, Cc,
                                                          C.c_void_p(out), Ho, Wo))

    def kernel_reconstruct(self, V, H, W, depth=0, pose_encoding=0, points_in_camera=0, quaternion=0, translation=0,
                           conf=0, mask=0, foreground=0, cameras=0, points=0, conf_out=0):
        ptrs = [depth, pose_encoding, points_in_camera, quaternion, translation, conf, mask, foreground, cameras,
                points, conf_out]
        self.check(self._lib.splat_kernel_reconstruct(self.handle, V, H, W, *[C.c_void_p(x or 0) for x in ptrs]))


def reference_ma_spec() -> dict:
    s = MaSpecC()
    lib().splat_ma_reference_spec(C.byref(s))
    return {name: (list(getattr(s, name)) if name in ("hooks", "dpt_dims") else getattr(s, name))
            for name, _ in MaSpecC._fields_}


def _check_free(rc: int):
    if rc != OK:
        raise SplatError(rc, lib().splat_last_error(None).decode())


def da3_model_input_size(width: int, height: int):
    """depthanything3-rs/src/preprocess.rs:36-45: ((bounded w, h), (w, h) in patch multiples)."""
    v = [C.c_int() for _ in range(4)]
    _check_free(lib().splat_da3_input_size(width, height, *[C.byref(x) for x in v]))
    return (v[0].value, v[1].value), (v[2].value, v[3].value)


def da3_model_inputs_size(sizes):
    """The common (W, H) of preprocess.rs:86-123 for images of sizes [(w, h)]."""
    d = [da3_model_input_size(w, h)[1] for w, h in sizes]
    return min(x[0] for x in d), min(x[1] for x in d)


def ma_input_size(sizes):
    """mapanything-rs/src/preprocess.rs:33-41 for images of sizes [(w, h)]: (W, H)."""
    ws = np.array([w for w, _ in sizes], np.int32)
    hs = np.array([h for _, h in sizes], np.int32)
    W, H = C.c_int(), C.c_int()
    _check_free(lib().splat_ma_input_size(len(sizes), _ptr(ws), _ptr(hs), C.byref(W), C.byref(H)))
    return W.value, H.value
