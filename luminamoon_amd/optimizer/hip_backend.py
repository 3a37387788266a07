"""ctypes binding of libluminav_hip.so (C ABI in include/luminav_hip.h) for ROCm tensors.

This module is the whole device path of the optimizer: it turns a list of PyTorch-ROCm tensors
into `lv_tensor` descriptors and calls `lv_step_multi` on the current stream. It replaces the
reference's per-tensor Triton dispatch `LuminaVGpuMixin._step_gpu_group`
(python/luminamoon/optimizer/gpu_backend.py:2603-2733). There is no fallback: if the shared
library is missing the step raises.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading
from typing import Any, Dict, List, Optional, Sequence

import numpy as np
import torch

_LIB_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib")
LIB_PATH = os.path.join(_LIB_DIR, "libluminav_hip.so")

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
BUFFER_CODES = {1: 1, 2: 2, "T1": 3, "T2": 4}

STATUS_NAMES = {0: "SUCCESS", -1: "NULL_POINTER", -2: "NO_DRIVER", -3: "INVALID_CONFIG", -4: "EXECUTION_FAILED"}


class LvConfig(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("tau", ctypes.c_float),
        ("lam", ctypes.c_float),
        ("cautious_clamp_min", ctypes.c_float),
        ("bound_ratio", ctypes.c_float),
        ("ema_decay", ctypes.c_float),
        ("buffer", ctypes.c_int32),
        ("cautious", ctypes.c_int32),
        ("stochastic_rounding", ctypes.c_int32),
        ("bound", ctypes.c_int32),
        ("bound_type", ctypes.c_int32),
        ("master_weights", ctypes.c_int32),
        ("fused_single_pass", ctypes.c_int32),
        ("seed", ctypes.c_uint32),
    ]


class LvTensor(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("master_param", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("numel", ctypes.c_uint64),
        ("step", ctypes.c_uint64),
        ("param_index", ctypes.c_uint64),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("state_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("index_base", ctypes.c_uint64),
        ("inactive", ctypes.c_void_p),
        ("n_inactive", ctypes.c_uint64),
    ]


class LvStepRecord(ctypes.Structure):
    """lv_step_record: the device-side step counter and coefficients of graph launches."""
    _fields_ = [
        ("step", ctypes.c_uint64),
        ("c1", ctypes.c_float),
        ("c2", ctypes.c_float),
        ("c_sigma", ctypes.c_float),
        ("seed_base", ctypes.c_uint32),
        ("status", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


EXPORTED_SYMBOLS = (
    "lv_version", "lv_workspace_bytes", "lv_workspace_bytes_for", "lv_step_multi", "lv_step_multi_graph",
    "lv_step_multi_noalloc", "lv_step_f32", "lv_last_error",
    # the reference's standalone C API (luminav_triton_standalone.h:37-111)
    "luminav_triton_engine_create", "luminav_triton_engine_destroy", "luminav_triton_get_platform",
    "luminav_triton_get_arch", "luminav_triton_step_f32",
)

_lib: Optional[ctypes.CDLL] = None
_lib_lock = threading.Lock()

HOST_EXT_PATH = os.path.join(_LIB_DIR, "_lv_host.so")


def load_host_ext() -> Any:
    """The plans' data-pointer checks (_lv_host.so, built from csrc/host_ptrs.cpp), or None when it
    is not built (the optimizer then compares pointers in Python: same results, more host time)."""
    if not os.path.exists(HOST_EXT_PATH):
        return None
    try:
        import importlib.util

        spec = importlib.util.spec_from_file_location("_lv_host", HOST_EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        return mod
    except (ImportError, OSError):
        return None


class HipBackendUnavailable(RuntimeError):
    pass


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libluminav_hip.so and declare its signatures. Raises if it is not built."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise HipBackendUnavailable(
                f"LuminaV HIP backend not built: {path} is missing. Run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950) before stepping ROCm tensors."
            )
        L = ctypes.CDLL(path)
        L.lv_version.restype = ctypes.c_int
        L.lv_version.argtypes = []
        L.lv_workspace_bytes.restype = ctypes.c_size_t
        L.lv_workspace_bytes.argtypes = [ctypes.c_int]
        L.lv_workspace_bytes_for.restype = ctypes.c_size_t
        L.lv_workspace_bytes_for.argtypes = [ctypes.POINTER(LvConfig), ctypes.POINTER(LvTensor), ctypes.c_int]
        L.lv_step_multi.restype = ctypes.c_int
        L.lv_step_multi.argtypes = [
            ctypes.POINTER(LvConfig), ctypes.POINTER(LvTensor), ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_void_p,
        ]
        L.lv_step_multi_graph.restype = ctypes.c_int
        L.lv_step_multi_graph.argtypes = [ctypes.POINTER(LvConfig), ctypes.POINTER(LvTensor), ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        L.lv_step_multi_noalloc.restype = ctypes.c_int
        L.lv_step_multi_noalloc.argtypes = [ctypes.POINTER(LvConfig), ctypes.POINTER(LvTensor), ctypes.c_int,
                                            ctypes.c_void_p]
        f, P = ctypes.c_float, ctypes.c_void_p
        L.lv_step_f32.restype = ctypes.c_int
        L.lv_step_f32.argtypes = [P, P, P, P, P, P, ctypes.c_size_t, f, f, f, f, f, f, f, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, f, ctypes.c_uint64, ctypes.c_uint32, P]
        L.lv_last_error.restype = ctypes.c_char_p
        L.lv_last_error.argtypes = []
        L.luminav_triton_engine_create.restype = P
        L.luminav_triton_engine_create.argtypes = []
        L.luminav_triton_engine_destroy.restype = None
        L.luminav_triton_engine_destroy.argtypes = [P]
        L.luminav_triton_get_platform.restype = ctypes.c_char_p
        L.luminav_triton_get_platform.argtypes = [P]
        L.luminav_triton_get_arch.restype = ctypes.c_char_p
        L.luminav_triton_get_arch.argtypes = [P]
        L.luminav_triton_step_f32.restype = ctypes.c_int
        L.luminav_triton_step_f32.argtypes = [P, P, P, P, P, P, P, ctypes.c_size_t, f, f, f, f, f, f, f, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int, f, ctypes.c_uint64, ctypes.c_uint32]
        _lib = L
        return L


def make_config(group: Dict[str, Any]) -> LvConfig:
    """C config from a normalised param group (python/luminamoon/optimizer/luminav.py:1825-1846)."""
    return LvConfig(
        float(group["lr"]), float(group["betas"][0]), float(group["betas"][1]), float(group["eps"]),
        float(group["weight_decay"]), float(group["tau"]), float(group["lam"]), float(group["cautious_clamp_min"]),
        float(group["bound_ratio"]), float(group["ema_decay"]), BUFFER_CODES[group["buffer"]],
        int(bool(group["cautious"])), int(bool(group["stochastic_rounding"])), int(bool(group["bound"])),
        int(group["bound_type"]), int(group["master_weights"]), int(bool(group["fused_single_pass"])),
        int(group["seed"]) & 0xFFFFFFFF,
    )


class _Workspace:
    """Per-device workspace (cautious count slots, radial records), allocated zero-filled and
    grown to the largest call seen; every call leaves all of it zero again, so calls of any
    layout share it. A replaced buffer is kept, not freed: launches already queued (possibly on
    another stream, which torch's allocator would not wait for) may still use it. Growth at least
    doubles, so the kept buffers total less than the live one."""

    def __init__(self) -> None:
        self._bufs: Dict[Any, torch.Tensor] = {}
        self._kept: List[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        buf = self._bufs.get(device)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._kept.append(buf)
                nbytes = max(nbytes, 2 * buf.numel())
            # torch's caching allocator returns 512-byte aligned blocks (the library needs 256)
            buf = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
            self._bufs[device] = buf
        return buf

    def discard(self, device: torch.device) -> None:
        """Retires the device's buffer: after a failed launch its count slots may hold a partial
        launch's counts, so the next call starts from a fresh zero-filled one."""
        buf = self._bufs.pop(device, None)
        if buf is not None:
            self._kept.append(buf)


# lv_tensor packed little-endian: 6 pointers, numel, step, param_index, 4 x int32, index_base,
# inactive, n_inactive (layout checked against the header by tests/test_c_abi.py).
_TENSOR = struct.Struct("<6Q3Q4i3Q")
_STEP_OFFSET = 7 * 8   # byte offset of lv_tensor.step
assert _TENSOR.size % 8 == 0 and _STEP_OFFSET % 8 == 0
_GRAD_OFFSET = 1 * 8   # byte offset of lv_tensor.grad
_OK_DTYPES = frozenset(DTYPE_CODES)


class PreparedStep:
    """Validated, packed descriptors for one lv_step_multi call. Between steps the caller may
    swap a tensor's grad (same shape/dtype/device, contiguous; checked) and set step counters;
    everything else stays as validated."""

    __slots__ = ("buf", "items", "n", "device", "numels", "gdtypes", "index", "_steps", "_gptrs", "ws_need")

    def __init__(self, buf: bytearray, n: int, device: torch.device, numels: List[int], gdtypes: List[Any]):
        self.buf = buf
        self.items = (LvTensor * n).from_buffer(buf) if n else None
        # the step field of every record, as one strided u64 view of the packed buffer
        self._steps = np.frombuffer(buf, dtype=np.uint64)[_STEP_OFFSET // 8::_TENSOR.size // 8] if n else None
        # the grad pointer of every record, for re-pointing all grads at once (set_grads)
        self._gptrs = np.frombuffer(buf, dtype=np.uint64)[_GRAD_OFFSET // 8::_TENSOR.size // 8] if n else None
        self.n = n
        self.device = device
        self.numels = numels
        self.gdtypes = gdtypes
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.ws_need: Dict[bool, int] = {}  # workspace bytes, by whether the radial bound is on

    def set_grad(self, i: int, g: torch.Tensor) -> bool:
        """Point descriptor i at grad g; False (nothing changed) if g does not fit it."""
        if (g.dtype is not self.gdtypes[i] or not g.is_cuda or g.get_device() != self.index
                or g.numel() != self.numels[i] or not g.is_contiguous()):
            return False
        struct.pack_into("<Q", self.buf, i * _TENSOR.size + _GRAD_OFFSET, g.data_ptr())
        return True

    def set_grads(self, grads: Sequence[torch.Tensor], ptrs: Sequence[int]) -> bool:
        """Point every descriptor at its grad (ptrs[i] = grads[i].data_ptr()) after checking them
        all as set_grad does; False (nothing changed) if any does not fit."""
        idx = self.index
        for g, dt, n in zip(grads, self.gdtypes, self.numels):
            if (g is None or g.dtype is not dt or g.layout is not torch.strided or g.get_device() != idx
                    or g.numel() != n or not g.is_contiguous()):  # get_device() is -1 off the GPU
                return False
        self._gptrs[:] = ptrs
        return True

    def set_grad_record(self, rec: bytes) -> None:
        """Point every descriptor at the grad pointers of a packed native-endian uint64 record
        (already checked against the descriptors, as set_grads checks them)."""
        self._gptrs[:] = np.frombuffer(rec, dtype=np.uint64)

    def set_step(self, i: int, step: int) -> None:
        struct.pack_into("<Q", self.buf, i * _TENSOR.size + _STEP_OFFSET, int(step))

    def set_steps(self, steps: Sequence[int]) -> None:
        """Step counter of every descriptor at once (len(steps) == n)."""
        self._steps[:] = steps


# The current device and its current stream's raw handle, read each step. torch's own C entry
# points skip the Python wrappers' argument handling (about 8 us per step on the cfg2 host path).
_get_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream_handle(index: int) -> int:
    if _raw_stream is not None:
        return int(_raw_stream(index))
    return torch.cuda.current_stream(index).cuda_stream


class HipStepper:
    """Runs one optimizer step for a list of same-device tensors through lv_step_multi."""

    def __init__(self) -> None:
        self.workspace = _Workspace()

    def prepare(
        self,
        params: Sequence[torch.Tensor],
        grads: Sequence[torch.Tensor],
        exp_avgs: Sequence[torch.Tensor],
        exp_avg_sqs: Sequence[Optional[torch.Tensor]],
        master_params: Sequence[Optional[torch.Tensor]],
        scratches: Sequence[torch.Tensor],
        steps: Sequence[int],
        param_indices: Sequence[int],
        index_bases: Optional[Sequence[int]] = None,
        inactive: Optional[Sequence[Optional[torch.Tensor]]] = None,
    ) -> Optional[PreparedStep]:
        """Validates every tensor and packs the lv_tensor descriptors (see step())."""
        n = len(params)
        if n == 0:
            return None
        device = params[0].device
        if device.type != "cuda":
            raise RuntimeError(
                "LuminaV (MI355X build) steps ROCm device tensors only; got a tensor on "
                f"'{device}'. Move the model to the GPU before calling step()."
            )
        buf = bytearray(n * _TENSOR.size)
        numels: List[int] = []
        gdtypes: List[Any] = []
        for i in range(n):
            p, g, m = params[i], grads[i], exp_avgs[i]
            v, mp, sc = exp_avg_sqs[i], master_params[i], scratches[i]
            for name, t in (("param", p), ("grad", g), ("exp_avg", m), ("scratch", sc)):
                if t.device != device:
                    raise ValueError(f"LuminaV: {name} of param index {param_indices[i]} is on {t.device}, expected {device}.")
                if not t.is_contiguous():
                    raise ValueError(f"LuminaV: {name} of param index {param_indices[i]} must be contiguous.")
            for name, t in (("param", p), ("grad", g), ("exp_avg", m)):
                if t.dtype not in _OK_DTYPES:
                    raise ValueError(f"LuminaV: unsupported dtype {t.dtype} for {name} of param index {param_indices[i]}.")
            numel = p.numel()
            if g.numel() != numel or m.numel() != numel:
                raise ValueError(
                    f"Shape mismatch for param index {param_indices[i]}: param={numel}, grad={g.numel()}, exp_avg={m.numel()}."
                )
            if sc.dtype != torch.float32 or sc.numel() < 6:
                raise ValueError(f"LuminaV: scratch of param index {param_indices[i]} must be float32[6].")
            vp = 0
            if v is not None:
                if v.numel() != numel:
                    raise ValueError(
                        f"Shape mismatch for exp_avg_sq at param index {param_indices[i]}: expected {numel}, got {v.numel()}."
                    )
                if v.dtype != m.dtype:
                    raise ValueError(
                        f"DType mismatch between exp_avg ({m.dtype}) and exp_avg_sq ({v.dtype}) at param index {param_indices[i]}."
                    )
                if v.device != device or not v.is_contiguous():
                    raise ValueError(f"LuminaV: exp_avg_sq of param index {param_indices[i]} must be contiguous on {device}.")
                vp = v.data_ptr()
            mpp = 0
            if mp is not None:
                if mp.numel() != numel:
                    raise ValueError(
                        f"Shape mismatch for master_param at param index {param_indices[i]}: expected {numel}, got {mp.numel()}."
                    )
                if mp.dtype != torch.float32:
                    raise ValueError("Tensor/buffer 'master_param' must have dtype float32.")
                if mp.device != device or not mp.is_contiguous():
                    raise ValueError(f"LuminaV: master_param of param index {param_indices[i]} must be contiguous on {device}.")
                mpp = mp.data_ptr()
            ip, ni = 0, 0
            rng = inactive[i] if inactive is not None else None
            if rng is not None and rng.numel() > 0:
                if rng.dtype != torch.int64 or rng.dim() != 2 or rng.shape[1] != 2 or not rng.is_contiguous():
                    raise ValueError("LuminaV: inactive ranges must be a contiguous int64 tensor of shape [k, 2].")
                if rng.device != device:
                    raise ValueError(f"LuminaV: inactive ranges of param index {param_indices[i]} must be on {device}.")
                ip, ni = rng.data_ptr(), int(rng.shape[0])
            _TENSOR.pack_into(
                buf, i * _TENSOR.size, p.data_ptr(), g.data_ptr(), m.data_ptr(), vp, mpp, sc.data_ptr(), numel,
                int(steps[i]), int(param_indices[i]), DTYPE_CODES[p.dtype], DTYPE_CODES[g.dtype], DTYPE_CODES[m.dtype], 0,
                int(index_bases[i]) if index_bases is not None else 0, ip, ni,
            )
            numels.append(numel)
            gdtypes.append(g.dtype)
        return PreparedStep(buf, n, device, numels, gdtypes)

    def launch(self, group: Dict[str, Any], prep: Optional[PreparedStep]) -> None:
        """One lv_step_multi call over prepared descriptors, on the device's current stream."""
        if prep is None or prep.n == 0:
            return
        lib = load_library()
        cfg = make_config(group)
        radial = bool(cfg.bound) and cfg.bound_type == 1 and cfg.bound_ratio > 0.0
        need = prep.ws_need.get(radial)
        if need is None:
            need = prep.ws_need[radial] = int(lib.lv_workspace_bytes_for(ctypes.byref(cfg), prep.items, prep.n))
        ws = self.workspace.get(prep.device, need)
        if _get_device() == prep.index:
            stream = _current_stream_handle(prep.index)
            rc = lib.lv_step_multi(ctypes.byref(cfg), prep.items, prep.n, ws.data_ptr(), ws.numel(), stream)
        else:
            with torch.cuda.device(prep.device):
                stream = _current_stream_handle(prep.index)
                rc = lib.lv_step_multi(ctypes.byref(cfg), prep.items, prep.n, ws.data_ptr(), ws.numel(), stream)
        if rc != 0:
            msg = lib.lv_last_error().decode(errors="replace")
            if rc in (-1, -3):  # rejected before any launch: the workspace is untouched
                raise ValueError(f"LuminaV HIP step rejected the call ({STATUS_NAMES.get(rc, rc)}): {msg}")
            self.workspace.discard(prep.device)
            raise RuntimeError(f"LuminaV HIP step failed ({STATUS_NAMES.get(rc, rc)}): {msg}")

    def graph_workspace_bytes(self, group: Dict[str, Any], prep: PreparedStep) -> int:
        """Workspace bytes an lv_step_multi_graph call over prep needs with the group's options."""
        cfg = make_config(group)
        return int(load_library().lv_workspace_bytes_for(ctypes.byref(cfg), prep.items, prep.n))

    def graph_workspace(self, group: Dict[str, Any], prep: PreparedStep) -> torch.Tensor:
        """A zeroed workspace of its own for lv_step_multi_graph calls over prep (graph replays
        must not share the stepper's workspace with eager calls on other streams)."""
        return torch.zeros(max(self.graph_workspace_bytes(group, prep), 256), dtype=torch.uint8, device=prep.device)

    def launch_graph(self, group: Dict[str, Any], prep: PreparedStep, record: torch.Tensor,
                     workspace: torch.Tensor) -> None:
        """One lv_step_multi_graph call: the step count and coefficients come from the device step
        record (an int64[4] tensor on prep's device), which the call advances on the stream."""
        lib = load_library()
        cfg = make_config(group)
        with torch.cuda.device(prep.device):
            stream = _current_stream_handle(prep.index)
            rc = lib.lv_step_multi_graph(ctypes.byref(cfg), prep.items, prep.n, record.data_ptr(), workspace.data_ptr(),
                                         workspace.numel(), stream)
        if rc != 0:
            msg = lib.lv_last_error().decode(errors="replace")
            if rc in (-1, -3):
                raise ValueError(f"LuminaV HIP graph step rejected the call ({STATUS_NAMES.get(rc, rc)}): {msg}")
            raise RuntimeError(f"LuminaV HIP graph step failed ({STATUS_NAMES.get(rc, rc)}): {msg}")

    def step(
        self,
        group: Dict[str, Any],
        params: Sequence[torch.Tensor],
        grads: Sequence[torch.Tensor],
        exp_avgs: Sequence[torch.Tensor],
        exp_avg_sqs: Sequence[Optional[torch.Tensor]],
        master_params: Sequence[Optional[torch.Tensor]],
        scratches: Sequence[torch.Tensor],
        steps: Sequence[int],
        param_indices: Sequence[int],
        index_bases: Optional[Sequence[int]] = None,
        inactive: Optional[Sequence[Optional[torch.Tensor]]] = None,
    ) -> None:
        """index_bases: global element offset of each tensor when it is a shard of a larger
        tensor (stochastic-rounding offsets continue from there); None = all 0.
        inactive: per tensor, None or an int64 device tensor of shape [k, 2] holding sorted,
        disjoint [begin, end) element ranges whose elements count in the statistics with a zero
        gradient but are not written (a fused bucket's grad=None slices)."""
        load_library()
        self.launch(group, self.prepare(params, grads, exp_avgs, exp_avg_sqs, master_params, scratches, steps,
                                        param_indices, index_bases, inactive))


def device_info() -> Dict[str, Any]:
    info: Dict[str, Any] = {"hip_backend_built": os.path.exists(LIB_PATH)}
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        info["gpu_device_name"] = props.name
        info["gpu_arch"] = getattr(props, "gcnArchName", None)
        info["compute_units"] = props.multi_processor_count
        info["hbm_bytes"] = props.total_memory
    else:
        info["gpu_device_name"] = None
    return info
