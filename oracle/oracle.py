"""ctypes wrapper around the C oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the
checker. The product package (luminamoon_amd) never imports it.

The oracle follows the reference's Rust CPU path (luminav-core + python_ffi/worker.rs); see
luminav_oracle.c for the per-function citations.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LVO_LIB_OVERRIDE lets the mutation test point the pins at a deliberately broken build.
_LIB_PATH = os.environ.get("LVO_LIB_OVERRIDE") or os.path.join(_HERE, "_build", "libluminav_oracle.so")

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
BUFFER_CODES = {1: 1, 2: 2, "T1": 3, "T2": 4}


class LvoConfig(ctypes.Structure):
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


class LvoTensor(ctypes.Structure):
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
    ]


_lib: Optional[ctypes.CDLL] = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    if os.environ.get("LVO_LIB_OVERRIDE"):
        return _LIB_PATH
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        f, i32, u32, u64, u16 = ctypes.c_float, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint16
        P = ctypes.c_void_p
        sigs = {
            "lvo_prng": (i32, [i32, i32]),
            "lvo_derive_kernel_seeds": (None, [u32, u64, u64, ctypes.POINTER(i32), ctypes.POINTER(i32)]),
            "lvo_derive_variance_seed": (i32, [i32]),
            "lvo_sanitize_gradient": (f, [f]),
            "lvo_tanh_pade": (f, [f]),
            "lvo_f32_to_f16_bits_rne": (u16, [f]),
            "lvo_f16_bits_to_f32": (f, [u16]),
            "lvo_sr_fp16_bits": (u16, [f, i32, i32]),
            "lvo_sr_fp16": (f, [f, i32, i32]),
            "lvo_rne_fp16": (f, [f]),
            "lvo_sr_bf16_bits": (u16, [f, i32, i32]),
            "lvo_sr_bf16": (f, [f, i32, i32]),
            "lvo_rne_bf16": (f, [f]),
            "lvo_quantize": (f, [f, i32, i32, i32, i32]),
            "lvo_bias_correction": (None, [u64, f, f, f, f, ctypes.POINTER(f)]),
            "lvo_t2_sigma_coeff": (f, [u64, f, f]),
            "lvo_powi": (ctypes.c_double, [ctypes.c_double, i32]),
            "lvo_cautious_scale": (f, [f, f, f]),
            "lvo_radial_scale": (f, [f, f, f, f, f]),
            "lvo_radial_scale_t2": (f, [f, f, f, f, f]),
            "lvo_coordinate_bound": (f, [f, f, f]),
            "lvo_coordinate_bound_t2": (f, [f, f, f]),
            "lvo_fp16_safety_bound": (f, [f, f]),
            "lvo_fp16_safety_bound_t2": (f, [f, f]),
            "lvo_update_post_step_ema": (None, [ctypes.POINTER(f), f, ctypes.POINTER(LvoConfig), i32]),
            "lvo_u64_to_f32": (f, [u64]),
            "lvo_set_radial_sum_mode": (None, [i32]),
            "lvo_set_backend": (i32, [i32]),
            "lvo_backend": (i32, []),
            "lvo_radial_sum_mode": (i32, []),
            "lvo_validate_config": (ctypes.c_int, [ctypes.POINTER(LvoConfig)]),
            "lvo_step_multi": (ctypes.c_int, [ctypes.POINTER(LvoConfig), ctypes.POINTER(LvoTensor), ctypes.c_int, ctypes.c_int]),
            "lvo_last_error": (ctypes.c_char_p, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _ = P
        _lib = L
    return _lib


@contextlib.contextmanager
def radial_sum_f64():
    """Inside the block the oracle adds the radial squares in f64 and rounds to f32 once (the
    HIP kernels' order-independent sum) instead of the scalar core's f32 lane order."""
    L = lib()
    old = L.lvo_radial_sum_mode()
    L.lvo_set_radial_sum_mode(1)
    try:
        yield
    finally:
        L.lvo_set_radial_sum_mode(old)


BACKEND_SCALAR, BACKEND_AVX512 = 0, 1


def avx512_available() -> bool:
    """True when this CPU runs the AVX-512 chunk kernels (avx512f/dq/bw/vl + fma)."""
    L = lib()
    old = L.lvo_backend()
    ok = L.lvo_set_backend(BACKEND_AVX512) == 0
    L.lvo_set_backend(old)
    return ok


@contextlib.contextmanager
def backend(which: int):
    """Inside the block the oracle runs its chunks on `which`: BACKEND_SCALAR (the scalar core,
    the default) or BACKEND_AVX512 (the restatement of luminav-simd's AVX-512 kernels)."""
    L = lib()
    old = L.lvo_backend()
    if L.lvo_set_backend(int(which)) != 0:
        raise RuntimeError(L.lvo_last_error().decode())
    try:
        yield
    finally:
        L.lvo_set_backend(old)


def make_config(
    lr: float = 3e-4,
    betas=(0.9, 0.999),
    eps: float = 1e-8,
    weight_decay: float = 0.08,
    tau: float = 0.8,
    lam: float = 0.3,
    cautious: bool = True,
    cautious_clamp_min: float = 0.5,
    buffer=2,
    stochastic_rounding: bool = True,
    bound: bool = True,
    bound_type: int = 2,
    bound_ratio: float = 0.05,
    master_weights: int = 0,
    fused_single_pass: bool = True,
    ema_decay: Optional[float] = None,
    seed: int = 1337,
) -> LvoConfig:
    """Config with the reference defaults (config.rs:297-321); floats round to f32 like
    python_ffi/config_parser.rs (`extract::<f32>`)."""
    code = BUFFER_CODES[buffer]
    if ema_decay is None:
        ema_decay = 0.95 if code in (1, 3) else 0.80
    return LvoConfig(
        lr, betas[0], betas[1], eps, weight_decay, tau, lam, cautious_clamp_min, bound_ratio, ema_decay,
        code, int(bool(cautious)), int(bool(stochastic_rounding)), int(bool(bound)), int(bound_type),
        int(master_weights), int(bool(fused_single_pass)), int(seed) & 0xFFFFFFFF,
    )


def _ptr(a) -> Optional[int]:
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        assert a.flags.c_contiguous
        return a.ctypes.data
    # torch CPU tensor
    assert a.is_contiguous() and a.device.type == "cpu"
    return a.data_ptr()


def _dtype_code(a) -> int:
    s = str(a.dtype)
    if "bfloat16" in s:
        return DTYPE_BF16
    if "float16" in s:
        return DTYPE_F16
    if "float32" in s:
        return DTYPE_F32
    if s in ("uint16",):  # numpy arrays holding bf16 bits
        return DTYPE_BF16
    raise ValueError(f"unsupported dtype {s}")


def step(
    cfg: LvoConfig,
    params: Sequence,
    grads: Sequence,
    exp_avgs: Sequence,
    exp_avg_sqs: Sequence,
    master_params: Sequence,
    scratches: Sequence,
    steps: Sequence[int],
    param_indices: Sequence[int],
    threads: int = 1,
    dtypes: Optional[Sequence[tuple]] = None,
    index_bases: Optional[Sequence[int]] = None,
) -> None:
    """In-place oracle step over host buffers (numpy arrays or CPU torch tensors).

    `dtypes`, when given, is a list of (param_dtype, grad_dtype, state_dtype) codes per item
    (needed for numpy uint16 arrays that hold bf16 or fp16 bits)."""
    n = len(params)
    items = (LvoTensor * max(n, 1))()
    for i in range(n):
        p, g, m = params[i], grads[i], exp_avgs[i]
        v = exp_avg_sqs[i]
        mp = master_params[i]
        sc = scratches[i]
        numel = int(p.numel() if hasattr(p, "numel") and callable(p.numel) else p.size)
        if dtypes is not None:
            pd, gd, sd = dtypes[i]
        else:
            pd, gd, sd = _dtype_code(p), _dtype_code(g), _dtype_code(m)
        items[i] = LvoTensor(
            _ptr(p), _ptr(g), _ptr(m), _ptr(v), _ptr(mp), _ptr(sc), numel, int(steps[i]),
            int(param_indices[i]), pd, gd, sd, 0, int(index_bases[i]) if index_bases is not None else 0,
        )
    rc = lib().lvo_step_multi(ctypes.byref(cfg), items, n, int(threads))
    if rc != 0:
        raise RuntimeError(f"oracle step failed ({rc}): {lib().lvo_last_error().decode()}")
