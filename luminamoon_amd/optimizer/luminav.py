"""LuminaV optimizer: the drop-in `LuminaV(params, ...)` / `step()` surface over the HIP backend.

Mirrors the reference class python/luminamoon/optimizer/luminav.py:
  - constructor, defaults and alias normalisation with the same error strings (:175-470, :472-761);
  - bounded contiguous bucket fusion with zero-copy views (:763-952) and its re-sync (:1293-1374);
  - lazy per-parameter state allocation and step counting (:1665-1798);
  - step routing, fused-bucket stepping with grad=None isolation (:1376-1606);
  - state_dict / load_state_dict format (:1030-1292).
The device work is one call of the C ABI lv_step_multi per (group, device) through
hip_backend.HipStepper; there is no per-tensor kernel loop and no CPU compute fallback.

Deliberate difference (the state-buffer allocation the MI355X path changes): 16-bit params get
fp32 exp_avg / exp_avg_sq by default (`state_precision="fp32"`), which is what the reference's
Rust core supports (python_ffi/mod.rs:57-125) and what the 7B bf16 bucket needs (12 B/param);
`state_precision="param"` restores the reference Python default (state in the param dtype
unless master_weights="full", luminav.py:1668-1672).
"""
from __future__ import annotations

import functools
import logging
import math
import operator
import struct
import warnings
import weakref
from collections import defaultdict
from itertools import repeat
from typing import Any, Callable, Dict, List, Optional, Set, Tuple, Union

import torch
from torch.optim import Optimizer
from torch.optim import optimizer as _torch_optimizer

from . import hip_backend
from .constants import (
    DEFAULT_BETAS,
    DEFAULT_BOUND_RATIO,
    DEFAULT_BUCKET_CAP_MB,
    DEFAULT_CAUTIOUS_CLAMP_MIN,
    DEFAULT_EPS,
    DEFAULT_FUSE_TENSORS,
    DEFAULT_FUSED_SINGLE_PASS,
    DEFAULT_GPU_DISPATCH_THRESHOLD,
    DEFAULT_LAM,
    DEFAULT_LR,
    DEFAULT_OPTIMIZER_SEED,
    DEFAULT_PREWARM_JIT,
    DEFAULT_STATE_PRECISION,
    DEFAULT_TAU,
    DEFAULT_WEIGHT_DECAY,
    TEMP_STATE_DICT_KEYS,
    VALID_BOUND_TYPE_CANDIDATES,
    VALID_BUFFER_CANDIDATES,
    VALID_EXECUTION_MODE_CANDIDATES,
    VALID_MASTER_WEIGHTS_CANDIDATES,
    VALID_STATE_PRECISION_CANDIDATES,
)
from .validation import is_valid_number, suggest_closest, validate_supported_dtype
from .version import (
    DEFAULT_LUMINAV_VERSION,
    SUPPORTED_VERSIONS,
    HybridVersionMethod,
    get_capabilities,
    validate_version,
)

logger = logging.getLogger("LuminaV")

_BUFFER_ERR = "LuminaV only supports buffer=1 (Single-Buffer TD-CLM) or buffer=2 (Dual-Buffer CLM)."
_SCRATCH_INIT = (0.0, 0.0, 0.0, 1.0, 1.0, 0.0)


def _new_scratch(device: torch.device) -> torch.Tensor:
    """ScratchBuffer::new() (luminav-core/src/state.rs:17-23)."""
    return torch.tensor(_SCRATCH_INIT, dtype=torch.float32, device=device)


# --------------------------------------------------------------------- fp16-container state codecs
# An fp16 *state* container holds bfloat16 bits (worker.rs:107-113, luminav.py:1096-1101).

def _decode_state_f32(buf: torch.Tensor) -> torch.Tensor:
    if buf.dtype == torch.float16:
        return buf.contiguous().view(torch.bfloat16).float()
    return buf.float()


def _encode_bf16_bits_rne(val: torch.Tensor) -> torch.Tensor:
    """f32 -> bf16 bits with the reference's RNE (prng.rs:162-178: overflow clamps to max finite)."""
    bits = val.contiguous().float().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    absb = bits & 0x7FFFFFFF
    sign = bits & 0x80000000
    lsb = (absb >> 16) & 1
    rnd = (absb + 0x7FFF + lsb) & 0xFFFF0000
    rnd = torch.minimum(rnd, torch.full_like(rnd, 0x7F7F0000))
    out = sign | rnd
    nan = absb > 0x7F800000
    out = torch.where(nan, (bits | 0x00400000) & 0xFFFF0000, out)
    hi = (out >> 16).to(torch.int32)
    hi = torch.where(hi >= 0x8000, hi - 0x10000, hi).to(torch.int16)
    return hi.view(torch.bfloat16)


def _convert_state_buffer(src: torch.Tensor, device: torch.device, target: torch.dtype,
                          fp16_is_bf16_bits: bool = True) -> torch.Tensor:
    """Move a state buffer to `device`/`target`, honouring fp16 containers of bf16 bits
    (reference luminav.py:124-146)."""
    buf = src.to(device=device).contiguous()
    if src.dtype == target:
        if src.dtype == torch.float16 and not fp16_is_bf16_bits:
            return _encode_bf16_bits_rne(buf.float()).view(torch.float16)
        return buf.clone()
    if src.dtype == torch.float16 or target == torch.float16:
        val = _decode_state_f32(buf) if (src.dtype != torch.float16 or fp16_is_bf16_bits) else buf.float()
        if target == torch.float16:
            return _encode_bf16_bits_rne(val).view(torch.float16)
        return val.to(dtype=target).contiguous()
    return buf.to(dtype=target).contiguous()


# --------------------------------------------------------------------- bucket buffers in HBM

_ARENA_ALIGN = 2 << 20  # every buffer of a bucket starts on a 2 MiB boundary of its allocation


class _ArenaPart:
    """One buffer of a bucket's device allocation, as an object that torch.as_tensor wraps without
    a copy (the CUDA array interface). The tensor it makes has a storage of its own, exactly the
    buffer's bytes (so torch.save of a model whose params live in a bucket writes only the params),
    and keeps the whole allocation alive through this object."""

    __slots__ = ("arena", "__cuda_array_interface__")

    def __init__(self, arena: torch.Tensor, offset: int, nbytes: int) -> None:
        self.arena = arena
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1",
                                         "data": (arena.data_ptr() + offset, False), "version": 2}


def _bucket_buffers(device: torch.device, specs: List[Tuple[str, torch.dtype, int]]) -> Dict[str, torch.Tensor]:
    """A bucket's flat buffers, in the order given. On a GPU they are laid out back to back, each on
    a 2 MiB boundary, in ONE allocation. The step streams these buffers in lockstep (element i of
    p, g, m and v at once). In physically fresh HBM (the first large allocations of a process on a
    freshly started device), separately allocated buffers ran the 6.7e9-element T2 step 4-7%
    slower than the same buffers allocated later in the process. Packed in the order p|g|m|v, in
    the same fresh memory, it ran within 2.5% of the later allocations; the order m|p|v|g of the
    same pack ran 5.5% slower than p|g|m|v. Elsewhere the layout is neutral.
    The parts' storages are not blocks of torch's caching allocator: `record_stream` on a part does
    not reach the allocation, which the allocator may reuse once the last part is freed (code that
    uses bucket tensors on a side stream keeps them alive until that stream is done with them)."""
    if device.type != "cuda":
        return {name: torch.empty(n, dtype=dt, device=device) for name, dt, n in specs}
    offs, off = [], 0
    for _, dt, n in specs:
        offs.append(off)
        off += (n * dt.itemsize + _ARENA_ALIGN - 1) // _ARENA_ALIGN * _ARENA_ALIGN
    arena = torch.empty(off + _ARENA_ALIGN, dtype=torch.uint8, device=device)
    base = (-arena.data_ptr()) % _ARENA_ALIGN
    out: Dict[str, torch.Tensor] = {}
    for (name, dt, n), o in zip(specs, offs):
        part = torch.as_tensor(_ArenaPart(arena, base + o, n * dt.itemsize), device=device)
        out[name] = part.view(dt)
    return out


_dict_set = dict.__setitem__
_get_grad = operator.attrgetter("grad")
_data_ptr = torch.Tensor.data_ptr

# Data-pointer records of the cached step plans: _ptr_record(tensors) records where a list of
# tensors' data is, _same_ptrs(tensors, record) tells whether it is still there (False for any
# entry that is not a tensor), _pack_ptrs(ints) makes a record from pointers. One C loop each
# when _lv_host.so is built, Python maps otherwise.
_host = hip_backend.load_host_ext()
# One C call for all of a step's checks of a plan whose every param has a grad, and one for its
# step counters (None without _lv_host.so, or with an older build of it).
_grad_record = getattr(_host, "grad_record", None)
_advance = getattr(_host, "advance", None)
if _host is not None:
    _ptr_record = _host.ptrs
    _same_ptrs = _host.same_ptrs

    def _pack_ptrs(ptrs: List[int]) -> bytes:
        return struct.pack(f"={len(ptrs)}Q", *ptrs)
else:
    def _ptr_record(tensors: List[Any]) -> List[int]:
        return list(map(_data_ptr, tensors))

    def _same_ptrs(tensors: List[Any], record: List[int]) -> bool:
        try:
            return list(map(_data_ptr, tensors)) == record
        except (AttributeError, TypeError):  # an entry that is not a tensor (a grad of None)
            return False

    def _pack_ptrs(ptrs: List[int]) -> List[int]:
        return list(ptrs)
_profiler_enabled = getattr(torch._C._autograd, "_profiler_enabled", lambda: True)


class _ParamState(dict):
    """One parameter's state dict. Replacing or removing any entry other than "step" (for example
    `opt.state[p]["exp_avg"] = t`, as device-moving helpers do) tells the optimizer: its cached
    step plans hold the state tensors' device pointers and are dropped."""

    __slots__ = ("_owner",)

    def __init__(self, owner: "weakref.ref", *args: Any, **kwargs: Any) -> None:
        dict.__init__(self, *args, **kwargs)
        self._owner = owner

    def _changed(self) -> None:
        opt = self._owner()
        if opt is not None:
            opt._invalidate_plans()

    def __setitem__(self, key: Any, value: Any) -> None:
        if key != "step":
            self._changed()
        else:  # a step counter set from outside: plans re-read the counters
            opt = self._owner()
            if opt is not None:
                opt._step_epoch += 1
        dict.__setitem__(self, key, value)

    def __delitem__(self, key: Any) -> None:
        self._changed()
        dict.__delitem__(self, key)

    def pop(self, key: Any, *default: Any) -> Any:
        if key in self:
            self._changed()
        return dict.pop(self, key, *default)

    def popitem(self) -> Any:
        self._changed()
        return dict.popitem(self)

    def clear(self) -> None:
        self._changed()
        dict.clear(self)

    def update(self, *args: Any, **kwargs: Any) -> None:
        self._changed()
        dict.update(self, *args, **kwargs)

    def setdefault(self, key: Any, default: Any = None) -> Any:
        if key not in self:
            self._changed()
        return dict.setdefault(self, key, default)

    def __ior__(self, other: Any) -> "_ParamState":
        self._changed()
        dict.update(self, other)
        return self

    def __reduce__(self) -> Any:  # pickles and copies as a plain dict
        return (dict, (dict(self),))


class _StateMap(defaultdict):
    """Optimizer.state holding _ParamState dicts. Replacing or removing a parameter's entry
    (`opt.state[p] = {...}`) tells the optimizer, like a change inside an entry does."""

    def __init__(self, owner: "LuminaV", src: Any = ()) -> None:
        self._owner = weakref.ref(owner)
        super().__init__(self._fresh)
        for k, v in dict(src).items():
            dict.__setitem__(self, k, self._wrap(v))

    def _fresh(self) -> _ParamState:
        return _ParamState(self._owner)

    def _wrap(self, v: Any) -> Any:
        if type(v) is dict:
            return _ParamState(self._owner, v)
        if isinstance(v, _ParamState):
            v._owner = self._owner
        return v

    def _changed(self) -> None:
        opt = self._owner()
        if opt is not None:
            opt._invalidate_plans()

    def __setitem__(self, key: Any, value: Any) -> None:
        self._changed()
        dict.__setitem__(self, key, self._wrap(value))

    def __delitem__(self, key: Any) -> None:
        self._changed()
        dict.__delitem__(self, key)

    def pop(self, key: Any, *default: Any) -> Any:
        if key in self:
            self._changed()
        return dict.pop(self, key, *default)

    def popitem(self) -> Any:
        self._changed()
        return dict.popitem(self)

    def clear(self) -> None:
        self._changed()
        dict.clear(self)

    def update(self, *args: Any, **kwargs: Any) -> None:
        self._changed()
        for k, v in dict(*args, **kwargs).items():
            dict.__setitem__(self, k, self._wrap(v))

    def setdefault(self, key: Any, default: Any = None) -> Any:
        if key not in self:
            self._changed()
            dict.__setitem__(self, key, self._wrap(default if default is not None else {}))
        return dict.__getitem__(self, key)

    def __reduce__(self) -> Any:  # pickles and copies as defaultdict(dict) of plain dicts
        return (defaultdict, (dict,), None, None, iter([(k, dict(v) if isinstance(v, dict) else v)
                                                         for k, v in self.items()]))


class LuminaV(Optimizer):
    """LuminaV optimizer (CLM `buffer=2`, TD-CLM `buffer=1`, Triangle family `"T1"`/`"T2"`) on MI355X.

    Same constructor and `step()` as the reference `luminamoon.LuminaV`; the update runs in
    hand-written HIP kernels (libluminav_hip.so) and is bitwise equal to the reference CPU
    implementation. Parameters must live on a ROCm device.
    """

    ALGORITHM_SPEC: str = DEFAULT_LUMINAV_VERSION
    ALGORITHM_MATH: str = DEFAULT_LUMINAV_VERSION
    _default_version: str = DEFAULT_LUMINAV_VERSION

    def __init__(
        self,
        params,
        lr: float = DEFAULT_LR,
        betas: Tuple[float, float] = DEFAULT_BETAS,
        eps: float = DEFAULT_EPS,
        weight_decay: float = DEFAULT_WEIGHT_DECAY,
        tau: float = DEFAULT_TAU,
        lam: float = DEFAULT_LAM,
        cautious: bool = True,
        cautious_clamp_min: float = DEFAULT_CAUTIOUS_CLAMP_MIN,
        buffer: Union[int, str] = 2,
        stochastic_rounding: bool = True,
        bound: bool = True,
        bound_type: Union[int, str] = "coordinate",
        bound_ratio: float = DEFAULT_BOUND_RATIO,
        master_weights: Union[bool, int, str] = "none",
        execution: Union[int, str] = "auto",
        fused_single_pass: bool = DEFAULT_FUSED_SINGLE_PASS,
        fuse_tensors: bool = DEFAULT_FUSE_TENSORS,
        bucket_cap_mb: float = DEFAULT_BUCKET_CAP_MB,
        prewarm_jit: bool = DEFAULT_PREWARM_JIT,
        ema_decay: Optional[Union[float, str]] = "auto",
        fsdp_sync: bool = False,
        seed: int = DEFAULT_OPTIMIZER_SEED,
        version: Optional[str] = None,
        spec: Optional[str] = None,
        state_precision: str = DEFAULT_STATE_PRECISION,
        capturable: bool = False,
    ):
        chosen = version if version is not None else spec
        self.version: str = validate_version(chosen if chosen is not None else self._default_version)
        defaults: Dict[str, Any] = dict(
            lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, tau=tau, lam=lam, cautious=cautious,
            cautious_clamp_min=cautious_clamp_min, buffer=buffer, stochastic_rounding=stochastic_rounding,
            bound=bound, bound_type=bound_type, bound_ratio=bound_ratio, master_weights=master_weights,
            execution=execution, fused_single_pass=fused_single_pass, fuse_tensors=fuse_tensors,
            bucket_cap_mb=bucket_cap_mb, prewarm_jit=prewarm_jit, ema_decay=ema_decay, fsdp_sync=fsdp_sync,
            seed=seed, version=self.version, state_precision=state_precision, capturable=capturable,
        )
        is_auto_ema = ema_decay is None or (isinstance(ema_decay, str) and ema_decay.strip().lower() == "auto")
        self._validate_and_normalize_group(defaults)
        if is_auto_ema:
            defaults["ema_decay"] = "auto"

        param_list = list(params)
        if len(param_list) == 0:
            raise ValueError("optimizer got an empty parameter list")
        first = param_list[0]
        first_p = (first.get("params") or [None])[0] if isinstance(first, dict) else first
        if not isinstance(first_p, torch.Tensor):
            raise TypeError(
                "LuminaV (MI355X build) optimizes torch.Tensor parameters on ROCm devices; "
                f"got {type(first_p).__name__}."
            )
        explicit_cap = bucket_cap_mb != DEFAULT_BUCKET_CAP_MB or any(
            isinstance(g, dict) and "bucket_cap_mb" in g for g in param_list
        )
        self._fused_buckets: List[Dict[str, Any]] = []
        super().__init__(param_list, defaults)

        self.seed = int(defaults["seed"])
        self.fuse_tensors: bool = bool(defaults["fuse_tensors"])
        self.bucket_cap_mb: float = float(defaults["bucket_cap_mb"])
        self.prewarm_jit: bool = bool(defaults["prewarm_jit"])
        self._stepper = hip_backend.HipStepper()
        # Packed descriptors of each unfused param group, reused while nothing but grads and step
        # counters changed (see _step_unfused); any state/param-group change bumps the epoch.
        self._unfused_plans: Dict[int, Dict[str, Any]] = {}
        self._plan_epoch = 0
        self._step_epoch = 0  # bumped when a step counter is set from outside
        # capturable groups: id(group) -> the group's device step record, workspace and descriptors
        self._graph_steps: Dict[int, Dict[str, Any]] = {}
        # records and workspaces of set-ups since replaced: a graph captured earlier still holds
        # their addresses, so they are never freed
        self._graph_retired: List[torch.Tensor] = []
        self.state = _StateMap(self, self.state)

        if any(bool(g.get("fuse_tensors", False)) for g in self.param_groups):
            self.fuse_tensors = True
            warnings.warn(
                "LuminaV: 'fuse_tensors=True' is designed for vision and image models (e.g., CNN, ViT) with "
                "many fragmented parameter layers. If you are training large language models (LLMs), "
                "it is recommended to keep 'fuse_tensors=False' to avoid unnecessary memory overhead.",
                UserWarning,
                stacklevel=2,
            )
            self._build_contiguous_buckets()
        elif explicit_cap:
            warnings.warn(
                f"LuminaV: 'bucket_cap_mb' was explicitly specified ({self.bucket_cap_mb} MB) "
                "but 'fuse_tensors' is False. Bounded bucket chunking only applies when parameter "
                "coalescing is enabled via 'fuse_tensors=True'. Parameters will be updated as "
                "standard individual tensors without chunked memory bounds.",
                UserWarning,
                stacklevel=2,
            )

    # ------------------------------------------------------------------ step wrapper

    @staticmethod
    def profile_hook_step(func: Callable) -> Callable:
        """torch.optim.Optimizer's step wrapper (global and per-optimizer pre/post hooks, a profiler
        range) with the profiler range opened only while a profiler runs: the range costs a few
        microseconds per step, a tenth of a small model's whole step here."""
        hooked = Optimizer.profile_hook_step(func)

        @functools.wraps(func)
        def wrapper(*args: Any, **kwargs: Any) -> Any:
            self = args[0]
            if (_profiler_enabled() or _torch_optimizer._global_optimizer_pre_hooks
                    or _torch_optimizer._global_optimizer_post_hooks or self._optimizer_step_pre_hooks
                    or self._optimizer_step_post_hooks):
                return hooked(*args, **kwargs)
            out = func(*args, **kwargs)
            self._optimizer_step_code()
            return out

        return wrapper

    # ------------------------------------------------------------------ versions

    def _set_version_inst(self, version: str) -> "LuminaV":
        self.version = validate_version(version)
        self.defaults["version"] = self.version
        for pg in self.param_groups:
            pg["version"] = self.version
        return self

    @classmethod
    def _set_version_cls(cls, version: str) -> str:
        cls._default_version = validate_version(version)
        return cls._default_version

    def _get_version_inst(self) -> str:
        return self.version

    @classmethod
    def _get_version_cls(cls) -> str:
        return cls._default_version

    set_version = HybridVersionMethod(_set_version_inst, _set_version_cls)
    setVersion = set_version
    set_spec = set_version
    setSpec = set_version
    get_version = HybridVersionMethod(_get_version_inst, _get_version_cls)
    getVersion = get_version
    get_spec = get_version
    getSpec = get_version
    get_math_version = get_version
    getMathVersion = get_version

    @property
    def spec(self) -> str:
        return self.version

    @property
    def math_version(self) -> str:
        return self.version

    @classmethod
    def _list_versions_cls(cls) -> List[str]:
        return list(SUPPORTED_VERSIONS)

    def _list_versions_inst(self) -> List[str]:
        return list(SUPPORTED_VERSIONS)

    list_versions = HybridVersionMethod(_list_versions_inst, _list_versions_cls)
    listVersions = list_versions

    @classmethod
    def _get_capabilities_cls(cls, version: Optional[str] = None) -> Dict[str, Any]:
        return get_capabilities(version if version is not None else cls._default_version)

    def _get_capabilities_inst(self, version: Optional[str] = None) -> Dict[str, Any]:
        return get_capabilities(version if version is not None else self.version)

    get_capabilities = HybridVersionMethod(_get_capabilities_inst, _get_capabilities_cls)
    getCapabilities = get_capabilities

    # ------------------------------------------------------------------ validation

    # Group keys that decide which state tensors a param has (and so the descriptors' pointers);
    # every other option is read into the launch config at each step.
    _LAYOUT_KEYS = ("buffer", "master_weights", "state_precision", "fuse_tensors", "fsdp_sync", "capturable")

    _SIG_KEYS = (
        "lr", "betas", "eps", "weight_decay", "tau", "lam", "cautious", "cautious_clamp_min", "buffer",
        "stochastic_rounding", "bound", "bound_type", "bound_ratio", "master_weights", "execution",
        "fused_single_pass", "fuse_tensors", "bucket_cap_mb", "prewarm_jit", "ema_decay", "fsdp_sync", "seed",
        "version", "state_precision", "capturable",
    )

    @staticmethod
    def _compute_group_sig(group: Dict[str, Any]) -> Tuple[Any, ...]:
        return tuple(map(group.get, LuminaV._SIG_KEYS))

    @staticmethod
    def _validate_and_normalize_group(group: Dict[str, Any]) -> None:
        """Validates and normalises one param group in place (reference luminav.py:472-761)."""
        lr, betas, eps = group["lr"], group["betas"], group["eps"]
        weight_decay, tau = group["weight_decay"], group["tau"]
        lam = group.get("lam", DEFAULT_LAM)
        cautious = group.get("cautious", True)
        cautious_clamp_min = group["cautious_clamp_min"]
        buffer = group["buffer"]
        bound = group.get("bound", True)
        bound_type = group["bound_type"]
        bound_ratio = group["bound_ratio"]
        master_weights = group["master_weights"]
        execution = group["execution"]
        fuse_tensors = group.get("fuse_tensors", DEFAULT_FUSE_TENSORS)
        prewarm_jit = group.get("prewarm_jit", DEFAULT_PREWARM_JIT)
        ema_decay = group.get("ema_decay", None)
        fsdp_sync = group.get("fsdp_sync", False)
        seed = group["seed"]
        state_precision = group.get("state_precision", DEFAULT_STATE_PRECISION)
        capturable = group.get("capturable", False)

        if not isinstance(capturable, bool):
            raise ValueError(f"Invalid capturable: {capturable!r}. Expected a boolean (True or False).")
        if capturable and fuse_tensors:
            raise ValueError(
                "LuminaV: capturable=True steps the group's parameters as separate tensors; set fuse_tensors=False."
            )
        if not isinstance(fuse_tensors, bool):
            raise ValueError(f"Invalid fuse_tensors: {fuse_tensors!r}. Expected a boolean (True or False).")
        if not isinstance(prewarm_jit, bool):
            raise ValueError(f"Invalid prewarm_jit: {prewarm_jit!r}. Expected a boolean (True or False).")
        if not is_valid_number(lr) or float(lr) < 0.0:
            raise ValueError(f"Invalid lr: {lr}. Expected a finite value in range [0.0, inf).")
        if not isinstance(betas, (tuple, list)) or len(betas) != 2:
            raise ValueError(
                f"Invalid betas: {betas}. Expected a 2-tuple (beta1, beta2) with values in range [0.0, 1.0)."
            )
        if not is_valid_number(betas[0]) or not (0.0 <= float(betas[0]) < 1.0):
            raise ValueError(f"Invalid beta1: {betas[0]}. Expected value in range [0.0, 1.0).")
        if not is_valid_number(betas[1]) or not (0.0 <= float(betas[1]) < 1.0):
            raise ValueError(f"Invalid beta2: {betas[1]}. Expected value in range [0.0, 1.0).")
        if not is_valid_number(eps) or float(eps) <= 0.0:
            raise ValueError(f"Invalid eps: {eps}. Expected value in range (0.0, inf).")
        if not is_valid_number(weight_decay) or float(weight_decay) < 0.0:
            raise ValueError(f"Invalid weight_decay: {weight_decay}. Expected value in range [0.0, inf).")
        if not is_valid_number(tau) or float(tau) <= 0.0:
            raise ValueError(f"Invalid tau: {tau}. Expected value in range (0.0, inf).")
        if not is_valid_number(lam) or float(lam) < 0.0:
            raise ValueError(f"Invalid lam: {lam}. Expected value in range [0.0, inf).")
        if not is_valid_number(cautious_clamp_min) or not (0.0 < float(cautious_clamp_min) <= 1.0):
            raise ValueError(
                f"Invalid cautious_clamp_min: {cautious_clamp_min}. Expected value in range (0.0, 1.0]."
            )
        if not is_valid_number(bound_ratio) or float(bound_ratio) <= 0.0:
            raise ValueError(f"Invalid bound_ratio: {bound_ratio}. Expected value in range (0.0, inf).")
        if isinstance(seed, bool) or not isinstance(seed, int) or seed < 0:
            raise ValueError(f"Invalid seed: {seed}. Expected a non-negative integer in range [0, 4294967295].")

        # buffer (luminav.py:552-587)
        if isinstance(buffer, bool):
            raise ValueError(f"Invalid buffer count: {buffer}. {_BUFFER_ERR}")
        if isinstance(buffer, int):
            if buffer not in (1, 2):
                raise ValueError(f"Invalid buffer count: {buffer}. {_BUFFER_ERR}")
            buf_val: Union[int, str] = int(buffer)
        elif isinstance(buffer, str):
            b = buffer.strip().lower()
            if b in ("1", "tdclm", "td-clm", "single"):
                buf_val = 1
            elif b in ("t2", "td-t2", "t2-clm", "td-dual", "triangle2", "clm-t2", "dual-t2"):
                buf_val = "T2"
            elif b in ("t1", "td-t1", "t1-clm", "triangle1", "td-clm-t1", "tdclm-t1"):
                buf_val = "T1"
            elif b in ("2", "dual", "clm"):
                buf_val = 2
            else:
                sug = suggest_closest(buffer, VALID_BUFFER_CANDIDATES, 2)
                hint = f" Did you mean '{sug}'?" if sug is not None else ""
                raise ValueError(f"Invalid buffer count: '{buffer}'. {_BUFFER_ERR}{hint}")
        else:
            raise ValueError(f"Invalid buffer count: {buffer}. {_BUFFER_ERR}")

        # version gates (luminav.py:589-605)
        gver = str(group.get("version", DEFAULT_LUMINAV_VERSION)).strip().lstrip("v")
        if gver in ("latest", "default", "reference", "canonical", "baseline"):
            gver = DEFAULT_LUMINAV_VERSION
        if gver in ("1.5.3", "1.5.4", "1.5.5") and buf_val in ("T1", "T2"):
            raise ValueError(
                f"LuminaV algorithm specification '{gver}' does not support Triangle Family buffer='{buffer}'. "
                f"Triangle Family tanh-free modes ('T1', 'T2') were introduced in LuminaV >= '1.6.0'. "
                f"To use '{buffer}', upgrade to version='1.6.0' (or omit version to use the default), or set buffer=2 / buffer=1."
            )
        if gver in ("1.5.3", "1.5.4") and bool(fuse_tensors):
            raise ValueError(
                f"LuminaV algorithm specification '{gver}' does not support contiguous bucket fusion (fuse_tensors=True). "
                f"Bucket fusion was introduced in LuminaV >= '1.5.5'. "
                f"To use fuse_tensors=True, upgrade to version >= '1.5.5' (or omit version to use default)."
            )

        # bound_type (luminav.py:607-633)
        if isinstance(bound_type, str):
            bt = bound_type.strip().lower()
            if bt in ("radial", "1"):
                bt_val = 1
            elif bt in ("coordinate", "2"):
                bt_val = 2
            elif bt in ("none", "0") and not bound:
                bt_val = 0
            else:
                sug = suggest_closest(bound_type, VALID_BOUND_TYPE_CANDIDATES, 3)
                hint = f" Did you mean '{sug}'?" if sug is not None else ""
                raise ValueError(f"Invalid bound_type: '{bound_type}'. Expected 'coordinate' or 'radial'.{hint}")
        elif not isinstance(bound_type, bool) and isinstance(bound_type, int):
            if bound_type not in (0, 1, 2):
                raise ValueError(f"Invalid bound_type: {bound_type}. Expected 'coordinate' or 'radial'.")
            bt_val = int(bound_type)
        else:
            raise ValueError(f"Invalid bound_type: {bound_type!r}. Expected 'coordinate' or 'radial'.")

        # master_weights (luminav.py:635-665)
        mw_err = "Expected False, 'none', 'semi', or 'full'."
        if isinstance(master_weights, bool):
            mw_val = 2 if master_weights else 0
        elif isinstance(master_weights, int):
            if master_weights not in (0, 1, 2):
                raise ValueError(f"Invalid master_weights: {master_weights}. {mw_err}")
            mw_val = int(master_weights)
        elif isinstance(master_weights, str):
            mw = master_weights.strip().lower()
            if mw in ("none", "false", "off", "0"):
                mw_val = 0
            elif mw in ("semi", "hybrid", "half", "1"):
                mw_val = 1
            elif mw in ("full", "true", "fp32", "masterweight", "2"):
                mw_val = 2
            else:
                sug = suggest_closest(master_weights, VALID_MASTER_WEIGHTS_CANDIDATES, 3)
                hint = f" Did you mean '{sug}'?" if sug is not None else ""
                raise ValueError(f"Invalid master_weights: '{master_weights}'. {mw_err}{hint}")
        else:
            raise ValueError(f"Invalid master_weights: {master_weights!r}. {mw_err}")

        # execution (luminav.py:667-701); every mode runs the HIP kernels on ROCm tensors.
        ex_err = "Expected 'auto', 'vulkan', 'simd', or 'scalar'."
        if isinstance(execution, str):
            ex = execution.strip().lower()
            table = {"auto": 0, "foreach": 0, "0": 0, "triton": 1, "1": 1, "single": 2, "2": 2, "vulkan": 3,
                     "3": 3, "simd": 4, "4": 4, "scalar": 5, "scalar_core": 5, "5": 5}
            if ex not in table:
                sug = suggest_closest(execution, VALID_EXECUTION_MODE_CANDIDATES, 3)
                hint = f" Did you mean '{sug}'?" if sug is not None else ""
                raise ValueError(f"Invalid execution mode: '{execution}'. {ex_err}{hint}")
            ex_val = table[ex]
        elif not isinstance(execution, bool) and isinstance(execution, int):
            if not 0 <= execution <= 5:
                raise ValueError(f"Invalid execution mode: {execution}. {ex_err}")
            ex_val = int(execution)
        else:
            raise ValueError(f"Invalid execution mode: {execution!r}. {ex_err}")

        # ema_decay (luminav.py:703-718)
        if ema_decay is None or (isinstance(ema_decay, str) and ema_decay.strip().lower() == "auto"):
            ema_val = 0.95 if buf_val in (1, "T1") else 0.80
        elif is_valid_number(ema_decay):
            ema_val = float(ema_decay)
            if not 0.0 < ema_val < 1.0:
                raise ValueError(f"Invalid ema_decay: {ema_decay}. Expected value in range (0.0, 1.0).")
        else:
            raise ValueError(
                f"Invalid ema_decay: {ema_decay!r}. Expected 'auto', None, or a float in range (0.0, 1.0)."
            )

        if not isinstance(state_precision, str) or state_precision.strip().lower() not in VALID_STATE_PRECISION_CANDIDATES:
            raise ValueError(f"Invalid state_precision: {state_precision!r}. Expected 'fp32' or 'param'.")

        if fsdp_sync and not (torch.distributed.is_available() and torch.distributed.is_initialized()):
            logger.warning(
                "LuminaV: fsdp_sync=True was specified, but torch.distributed is not initialized. "
                "Disabling fsdp_sync to prevent collective communication errors."
            )
            fsdp_sync = False
        if fsdp_sync and torch.distributed.get_world_size() > 1:
            # The reference all-reduces the per-tensor mask counts across ranks before the scale
            # (fsdp_sync.py:20-38). This build steps one GPU per process without that collective,
            # so a sharded run would silently use rank-local scales: refuse it instead.
            raise NotImplementedError(
                f"LuminaV: fsdp_sync=True across {torch.distributed.get_world_size()} ranks is not supported by "
                "this build (one GPU per process, no cross-rank scratch all-reduce)."
            )

        raw_cap = group.get("bucket_cap_mb", DEFAULT_BUCKET_CAP_MB)
        if raw_cap is None or not is_valid_number(raw_cap) or float(raw_cap) <= 0.0:
            raise ValueError(f"bucket_cap_mb must be a positive number, got: {raw_cap!r}")

        group.update(
            lr=float(lr), betas=(float(betas[0]), float(betas[1])), eps=float(eps), weight_decay=float(weight_decay),
            tau=float(tau), lam=float(lam), cautious=bool(cautious), cautious_clamp_min=float(cautious_clamp_min),
            buffer=buf_val, stochastic_rounding=bool(group.get("stochastic_rounding", True)), bound=bool(bound),
            bound_type=bt_val, bound_ratio=float(bound_ratio), master_weights=mw_val, execution=ex_val,
            fused_single_pass=bool(group.get("fused_single_pass", DEFAULT_FUSED_SINGLE_PASS)),
            fuse_tensors=bool(fuse_tensors), bucket_cap_mb=float(raw_cap), prewarm_jit=bool(prewarm_jit),
            ema_decay=ema_val, fsdp_sync=bool(fsdp_sync), seed=int(seed),
            state_precision=state_precision.strip().lower(), capturable=capturable,
        )
        group["_validated_sig"] = LuminaV._compute_group_sig(group)

    # ------------------------------------------------------------------ state policy

    @staticmethod
    def _state_dtype(p_dtype: torch.dtype, master_mode: int, precision: str) -> torch.dtype:
        if master_mode == 2 or p_dtype == torch.float32 or precision == "fp32":
            return torch.float32
        return p_dtype

    @staticmethod
    def _radial_active(group: Dict[str, Any]) -> bool:
        return bool(group.get("bound", True) and group.get("bound_type", 2) in (1, "radial")
                    and float(group.get("bound_ratio", 0.05)) > 0.0)

    # ------------------------------------------------------------------ bucket fusion

    @staticmethod
    def _partition_into_bounded_chunks(indexed_params: List[Tuple[int, Any]], cap_bytes: int) -> List[List[Tuple[int, Any]]]:
        """Cuts a run of params, in order, into buckets under cap_bytes. The cut rule is the
        reference's (luminav.py:763-786), since bucket boundaries fix each element's bucket offset
        and with it the stochastic-rounding stream: a param that would take a non-empty bucket
        past the cap opens the next bucket, so a param larger than the cap sits alone."""
        starts: List[int] = []
        fill = 0
        for k, (_, p) in enumerate(indexed_params):
            nbytes = int(p.numel() * p.element_size())
            if not starts or fill + nbytes > cap_bytes:  # the first param, or the open bucket is full
                starts.append(k)
                fill = 0
            fill += nbytes
        bounds = starts + [len(indexed_params)]
        return [list(indexed_params[a:b]) for a, b in zip(bounds, bounds[1:])]

    def _bucket_members(self, group: Dict[str, Any], claimed: Set[Any]) -> List[List[Tuple[int, Any]]]:
        """The group's buckets as lists of (param index, param): trainable non-empty params grouped
        by (device, dtype) in first-seen order, each run cut under the group's cap. A tensor
        already claimed (tied weights, or a param in an earlier group's bucket) is skipped, so its
        first occurrence owns the slice."""
        cap_bytes = int(float(group.get("bucket_cap_mb", DEFAULT_BUCKET_CAP_MB)) * (1 << 20))
        if cap_bytes <= 0:
            cap_bytes = int(DEFAULT_BUCKET_CAP_MB * (1 << 20))
        runs: Dict[Tuple[Any, Any], List[Tuple[int, Any]]] = {}
        for idx, p in enumerate(group["params"]):
            if not (isinstance(p, torch.Tensor) and p.requires_grad):
                continue
            validate_supported_dtype(p, "param")
            if p.numel() == 0:
                continue
            where = (p.device, p.data_ptr(), int(p.numel()))
            if id(p) in claimed or where in claimed:
                continue
            claimed.update((id(p), where))
            runs.setdefault((p.device, p.dtype), []).append((idx, p))
        return [chunk for run in runs.values() for chunk in self._partition_into_bounded_chunks(run, cap_bytes)]

    def _make_bucket(self, group: Dict[str, Any], members: List[Tuple[int, Any]]) -> Dict[str, Any]:
        """One bucket: flat p/g/m/v/master buffers and one scratch; each member's param, grad and
        state move into views of them (reference luminav.py:788-952 builds the same layout)."""
        dev, dt = members[0][1].device, members[0][1].dtype
        dual = group["buffer"] in (2, "T2")
        master_mode = int(group["master_weights"])
        sdt = self._state_dtype(dt, master_mode, group.get("state_precision", DEFAULT_STATE_PRECISION))
        numels = [int(p.numel()) for _, p in members]
        total = sum(numels)
        with_mp = master_mode > 0 and dt in (torch.float16, torch.bfloat16)
        specs = [("p", dt, total), ("g", dt, total), ("m", sdt, total)]
        specs += [("v", sdt, total)] if dual else []
        specs += [("mp", torch.float32, total)] if with_mp else []
        bufs = _bucket_buffers(dev, specs)
        for name in ("g", "m", "v"):
            if name in bufs:
                bufs[name].zero_()
        flats: Dict[str, Optional[torch.Tensor]] = {k: bufs.get(k) for k in ("p", "g", "m", "v", "mp")}
        parts = {k: (torch.split(f, numels) if f is not None else [None] * len(members)) for k, f in flats.items()}
        scratch = _new_scratch(dev)
        bucket = {
            "group": group, "device": dev, "dtype": dt, "state_dtype": sdt, "buf_count": group["buffer"],
            "master_mode": master_mode, "bucket_cap_mb": float(group.get("bucket_cap_mb", DEFAULT_BUCKET_CAP_MB)),
            "flat_p": flats["p"], "flat_g": flats["g"], "flat_m": flats["m"], "flat_v": flats["v"],
            "flat_mp": flats["mp"], "scratch": scratch, "slices": [], "step": 0,
        }
        if bucket["bucket_cap_mb"] <= 0:
            bucket["bucket_cap_mb"] = float(DEFAULT_BUCKET_CAP_MB)
        for k, (idx, p) in enumerate(members):
            view = {name: (part[k].view(p.shape) if part[k] is not None else None) for name, part in parts.items()}
            view["p"].copy_(p.detach())
            p.data = view["p"]
            if p.grad is not None:
                view["g"].copy_(p.grad.detach())
            p.grad = view["g"]
            if view["mp"] is not None:
                view["mp"].copy_(view["p"].float())
            st = self.state[p]
            # carry over existing state of the same size, converted to the bucket's state dtype
            for key, name, conv in (("exp_avg", "m", True), ("exp_avg_sq", "v", True), ("master_param", "mp", False)):
                old, dst = st.get(key), view[name]
                if dst is not None and isinstance(old, torch.Tensor) and old.numel() == dst.numel():
                    src = _convert_state_buffer(old, dev, sdt) if conv else old.to(device=dev, dtype=torch.float32)
                    dst.copy_(src.view(p.shape))
            if "step" in st:  # the bucket counts from the largest step seen so far
                seen = st["step"]
                bucket["step"] = max(bucket["step"], int(seen.item() if hasattr(seen, "item") else seen))
            old_sc = st.get("scratch")
            if isinstance(old_sc, torch.Tensor) and old_sc.numel() >= 6:
                scratch.copy_(old_sc.to(device=dev, dtype=torch.float32)[:6])
            st["step"] = bucket["step"]
            st["scratch"] = scratch
            st["buf_count"] = group["buffer"]
            for key, name in (("exp_avg", "m"), ("exp_avg_sq", "v"), ("master_param", "mp")):
                if view[name] is None:
                    st.pop(key, None)
                else:
                    st[key] = view[name]
            bucket["slices"].append((p, view["p"], view["g"], view["p"].data_ptr(), view["g"].data_ptr(), st, idx))
        return bucket

    def _build_contiguous_buckets(self, force_rebuild: bool = False) -> None:
        """Buckets for every fused group that has none yet (all of them with force_rebuild)."""
        if force_rebuild:
            self._fused_buckets.clear()
        built = {id(b["group"]) for b in self._fused_buckets}
        claimed: Set[Any] = set()
        for b in self._fused_buckets:
            for p, *_ in b["slices"]:
                claimed.add((p.device, p.data_ptr(), int(p.numel())))
        for group in self.param_groups:
            if id(group) in built or not group.get("fuse_tensors", False) or group.get("fsdp_sync", False):
                continue
            for members in self._bucket_members(group, claimed):
                self._fused_buckets.append(self._make_bucket(group, members))

    def _bucket_is_stale(self, b: Dict[str, Any]) -> bool:
        g = b["group"]
        return (not g.get("fuse_tensors", False) or g.get("fsdp_sync", False) or g.get("buffer", 2) != b["buf_count"]
                or int(g.get("master_weights", 0)) != int(b["master_mode"])
                or float(g.get("bucket_cap_mb", DEFAULT_BUCKET_CAP_MB)) != float(b["bucket_cap_mb"]))

    def _sync_or_rebuild_fused_buckets(self) -> None:
        """After load_state_dict or a change of bucket options: rebuilds every bucket when a fused
        group has none or a bucket no longer matches its group's options; otherwise moves each
        slice's (possibly replaced) param, grad and state tensors back into the bucket's views
        (reference luminav.py:1293-1374)."""
        with_buckets = {id(b["group"]) for b in self._fused_buckets}
        missing = any(g.get("fuse_tensors", False) and not g.get("fsdp_sync", False) and id(g) not in with_buckets
                      for g in self.param_groups)
        if missing or any(map(self._bucket_is_stale, self._fused_buckets)):
            self._build_contiguous_buckets(force_rebuild=True)
            return
        for b in self._fused_buckets:
            self._rebind_bucket(b)

    def _rebind_bucket(self, b: Dict[str, Any]) -> None:
        flats = {"exp_avg": b["flat_m"], "exp_avg_sq": b["flat_v"], "master_param": b["flat_mp"]}
        scratch = b["scratch"]
        step = int(b.get("step", 0))
        rebound = []
        off = 0
        for p, p_sl, g_sl, p_ptr, g_ptr, _, idx in b["slices"]:
            n = int(p.numel())
            if p.data_ptr() != p_ptr:
                p_sl.copy_(p.detach())
                p.data = p_sl
            if p.grad is not None and p.grad.data_ptr() != g_ptr:
                g_sl.copy_(p.grad.detach())
            p.grad = g_sl
            st = self.state[p]
            for key, flat in flats.items():
                cur = st.get(key)
                if flat is None or not isinstance(cur, torch.Tensor):
                    continue
                home = flat[off:off + n].view(p.shape)
                if cur.data_ptr() != home.data_ptr():
                    home.copy_(cur.detach())
                st[key] = home
            if "step" in st:  # the last slice's counter becomes the bucket's
                seen = st["step"]
                step = int(seen.item() if hasattr(seen, "item") else seen)
                st["step"] = step
            cur = st.get("scratch")
            if isinstance(cur, torch.Tensor) and cur.numel() >= 6:
                if cur.data_ptr() != scratch.data_ptr():
                    scratch.copy_(cur[:6])
                st["scratch"] = scratch
            rebound.append((p, p_sl, g_sl, p_ptr, g_ptr, st, idx))
            off += n
        b["slices"] = rebound
        b["step"] = step

    def _invalidate_plans(self) -> None:
        if hasattr(self, "_unfused_plans"):
            self._unfused_plans.clear()
            self._plan_epoch += 1


    def add_param_group(self, param_group: Dict[str, Any]) -> None:
        self._invalidate_plans()
        for name, default in self.defaults.items():
            param_group.setdefault(name, default)
        self._validate_and_normalize_group(param_group)
        super().add_param_group(param_group)
        if hasattr(self, "_stepper") and param_group.get("fuse_tensors", False):
            self.fuse_tensors = True
            self._build_contiguous_buckets()

    def zero_grad(self, set_to_none: bool = True) -> None:
        """Fused params keep their grad views into the bucket (reference luminav.py:973-1013)."""
        if self.fuse_tensors and self._fused_buckets:
            with torch.no_grad():
                fused_ids = set()
                for b in self._fused_buckets:
                    b["flat_g"].zero_()
                    for p, _, g_sl, _, g_ptr, _, _ in b["slices"]:
                        fused_ids.add(id(p))
                        if p.grad is not g_sl and (p.grad is None or p.grad.data_ptr() != g_ptr):
                            p.grad = g_sl
                for group in self.param_groups:
                    for p in group["params"]:
                        if id(p) in fused_ids or p.grad is None:
                            continue
                        if set_to_none:
                            p.grad = None
                        else:
                            if p.grad.grad_fn is not None:
                                p.grad.detach_()
                            else:
                                p.grad.requires_grad_(False)
                            p.grad.zero_()
            return
        super().zero_grad(set_to_none=set_to_none)

    @staticmethod
    def detect_hardware() -> Dict[str, Any]:
        info = {
            "simd_backend": None,
            "triton_aot_available": False,
            "triton_arch": None,
            "vulkan_available": False,
            "wave32_supported": False,
            "gpu_dispatch_threshold": DEFAULT_GPU_DISPATCH_THRESHOLD,
            "backend": "hip",
        }
        info.update(hip_backend.device_info())
        return info

    # ------------------------------------------------------------------ checkpoints

    def state_dict(self) -> Dict[str, Any]:
        """torch's state_dict in the reference's checkpoint format (luminav.py:1030-1115): no
        transient keys, no master copy for an fp32 param (the param is its own master), scratch
        accumulators zeroed, step counters as ints, and an fp16 state container tagged as holding
        bf16 bits."""
        raw = super().state_dict()
        own = {id(p) for g in self.param_groups for p in g["params"]}
        state = {k: (self._export_state(st, own) if isinstance(st, dict) else st) for k, st in raw.get("state", {}).items()}
        groups = [{k: v for k, v in g.items() if k != "_validated_sig"} for g in raw.get("param_groups", [])]
        return {"state": state, "param_groups": groups}

    @staticmethod
    def _export_state(st: Dict[str, Any], own: Set[int]) -> Dict[str, Any]:
        out: Dict[str, Any] = {}
        for key, val in st.items():
            if key in TEMP_STATE_DICT_KEYS or (key == "master_param" and id(val) in own):
                continue
            if not isinstance(val, torch.Tensor):
                out[key] = val
            elif key == "step":  # a capturable group's device counter
                out[key] = int(val.item())
            elif key == "scratch" and val.numel() >= 6:
                kept = val.detach().clone()
                kept[[0, 1, 2, 5]] = 0.0  # per-step accumulators; 3 and 4 are the EMA scales
                out[key] = kept
            else:
                out[key] = val.detach().clone()
        if any(isinstance(out.get(k), torch.Tensor) and out[k].dtype == torch.float16 for k in ("exp_avg", "exp_avg_sq")):
            out["_fp16_state_format"] = "bf16_bits"
        return out

    def load_state_dict(self, state_dict: Dict[str, Any]) -> None:
        """Loads state and re-normalises dtypes, scratch layout and buckets (reference luminav.py:1117-1292)."""
        self._invalidate_plans()
        raw_state = state_dict.get("state", {})
        saved_groups = state_dict.get("param_groups", [])
        raw_param_state: Dict[Any, Dict[str, Any]] = {}
        precision_of: Dict[int, str] = {}  # group position -> state precision of its saved state
        if len(self.param_groups) == len(saved_groups):
            for gi, (group, sg) in enumerate(zip(self.param_groups, saved_groups)):
                half_state: Set[bool] = set()
                for p, pid in zip(group["params"], sg.get("params", [])):
                    st = raw_state.get(pid)
                    if isinstance(st, dict):
                        raw_param_state[p] = {k: (v.detach().clone() if isinstance(v, torch.Tensor) else v) for k, v in st.items()}
                        m = st.get("exp_avg")
                        if p.dtype in (torch.float16, torch.bfloat16) and isinstance(m, torch.Tensor):
                            half_state.add(m.dtype in (torch.float16, torch.bfloat16))
                if "state_precision" not in sg and len(half_state) == 1:
                    # A checkpoint without this build's state_precision key (the reference's own
                    # format): keep the precision its 16-bit params' state was saved in. The
                    # reference stores that state in the param dtype unless master_weights="full"
                    # (python/luminamoon/optimizer/luminav.py:1666-1672).
                    precision_of[gi] = "param" if half_state.pop() else "fp32"
        super().load_state_dict(state_dict)
        for gi, group in enumerate(self.param_groups):
            if gi in precision_of:
                group["state_precision"] = precision_of[gi]
            for k, v in self.defaults.items():
                group.setdefault(k, v)
            self._validate_and_normalize_group(group)
            master_mode = int(group["master_weights"])
            buf_count = group["buffer"]
            precision = group.get("state_precision", DEFAULT_STATE_PRECISION)
            radial = self._radial_active(group)
            for p in group["params"]:
                if p not in self.state:
                    continue
                st = self.state[p]
                raw_st = raw_param_state.get(p, {})
                for tk in TEMP_STATE_DICT_KEYS:
                    st.pop(tk, None)
                if isinstance(st.get("step"), torch.Tensor):
                    st["step"] = int(st["step"].item())
                src_sc = raw_st.get("scratch") if isinstance(raw_st.get("scratch"), torch.Tensor) else st.get("scratch")
                sc = _new_scratch(p.device)
                if isinstance(src_sc, torch.Tensor):
                    old = src_sc.to(device=p.device, dtype=torch.float32).reshape(-1)[:6]
                    sc[: old.numel()].copy_(old)
                sc[:3].zero_()
                sc[5].zero_()
                if not group["cautious"]:
                    sc[3] = 1.0
                if not radial:
                    sc[4] = 1.0
                st["scratch"] = sc
                if master_mode == 0 or p.dtype == torch.float32:
                    st.pop("master_param", None)
                else:
                    src_mp = raw_st.get("master_param") if isinstance(raw_st.get("master_param"), torch.Tensor) else st.get("master_param")
                    if isinstance(src_mp, torch.Tensor):
                        st["master_param"] = src_mp.to(device=p.device, dtype=torch.float32).contiguous()
                    else:
                        st["master_param"] = p.detach().clone().float().contiguous()
                target = self._state_dtype(p.dtype, master_mode, precision)
                fp16_bits = (raw_st.get("_fp16_state_format") == "bf16_bits" or st.get("_fp16_state_format") == "bf16_bits"
                             or "scratch" in raw_st or "buf_count" in raw_st)
                st.pop("_fp16_state_format", None)
                for key in ("exp_avg", "exp_avg_sq"):
                    src = raw_st.get(key) if isinstance(raw_st.get(key), torch.Tensor) else st.get(key)
                    if isinstance(src, torch.Tensor):
                        st[key] = _convert_state_buffer(src, p.device, target, fp16_is_bf16_bits=fp16_bits)
                if not isinstance(st.get("exp_avg"), torch.Tensor):
                    st["exp_avg"] = torch.zeros_like(p, dtype=target, memory_format=torch.contiguous_format)
                if buf_count in (1, "T1"):
                    st.pop("exp_avg_sq", None)
                elif not isinstance(st.get("exp_avg_sq"), torch.Tensor):
                    st["exp_avg_sq"] = torch.zeros_like(p, dtype=target, memory_format=torch.contiguous_format)
                st["buf_count"] = buf_count
        self.fuse_tensors = any(bool(g.get("fuse_tensors", False)) for g in self.param_groups)
        if self.fuse_tensors:
            self._sync_or_rebuild_fused_buckets()
        else:
            self._fused_buckets.clear()
        self.state = _StateMap(self, self.state)
        self._invalidate_plans()

    # ------------------------------------------------------------------ step

    def _init_or_refresh_state(self, p: torch.Tensor, group: Dict[str, Any]) -> Dict[str, Any]:
        """Lazy state allocation and re-normalisation (reference luminav.py:1665-1790)."""
        buf_count = group["buffer"]
        master_mode = int(group["master_weights"])
        sdt = self._state_dtype(p.dtype, master_mode, group.get("state_precision", DEFAULT_STATE_PRECISION))
        state = self.state[p]
        if len(state) == 0:
            state["step"] = 0
            state["scratch"] = _new_scratch(p.device)
            state["exp_avg"] = torch.zeros_like(p, dtype=sdt, memory_format=torch.contiguous_format)
            if buf_count in (2, "T2"):
                state["exp_avg_sq"] = torch.zeros_like(p, dtype=sdt, memory_format=torch.contiguous_format)
            if master_mode > 0 and p.dtype in (torch.float16, torch.bfloat16):
                state["master_param"] = p.detach().clone().float().contiguous()
            state["buf_count"] = buf_count
            return state
        if master_mode > 0:
            if p.dtype == torch.float32:
                state.pop("master_param", None)
            elif state.get("master_param") is None:
                state["master_param"] = p.detach().clone().float().contiguous()
            elif state["master_param"].device != p.device or state["master_param"].dtype != torch.float32:
                state["master_param"] = state["master_param"].to(device=p.device, dtype=torch.float32)
        else:
            state.pop("master_param", None)
        sc = state.get("scratch")
        if not isinstance(sc, torch.Tensor) or sc.numel() < 6:
            new = _new_scratch(p.device)
            if isinstance(sc, torch.Tensor):
                new[: sc.numel()].copy_(sc.to(device=p.device, dtype=torch.float32))
            state["scratch"] = new
            state["buf_count"] = buf_count
        elif sc.device != p.device or sc.dtype != torch.float32:
            state["scratch"] = sc.to(device=p.device, dtype=torch.float32)
            state["buf_count"] = buf_count
        elif state.get("buf_count", buf_count) != buf_count:
            state["scratch"].copy_(torch.tensor(_SCRATCH_INIT, dtype=torch.float32))  # ParamState::ensure_buffer_mode
            state["buf_count"] = buf_count
        if "exp_avg" not in state:
            state["exp_avg"] = torch.zeros_like(p, dtype=sdt, memory_format=torch.contiguous_format)
        elif state["exp_avg"].device != p.device or state["exp_avg"].dtype != sdt:
            state["exp_avg"] = _convert_state_buffer(state["exp_avg"], p.device, sdt)
        if buf_count in (2, "T2"):
            if "exp_avg_sq" not in state:
                state["exp_avg_sq"] = torch.zeros_like(p, dtype=sdt, memory_format=torch.contiguous_format)
            elif state["exp_avg_sq"].device != p.device or state["exp_avg_sq"].dtype != sdt:
                state["exp_avg_sq"] = _convert_state_buffer(state["exp_avg_sq"], p.device, sdt)
        else:
            state.pop("exp_avg_sq", None)
        return state

    def step(self, closure: Optional[Callable[[], float]] = None, grads: Optional[Any] = None) -> Optional[float]:
        """One optimizer step over every param group (reference luminav.py:1376-1966), under
        no_grad like the reference's; a group stepped from its cached plan runs no tensor
        operation, so that path skips the no_grad context."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if type(self.state) is not _StateMap:  # replaced wholesale (assignment, unpickling)
            self.state = _StateMap(self, self.state)
            self._invalidate_plans()
        for group in self.param_groups:
            if group.get("_validated_sig") != self._compute_group_sig(group):
                self._validate_and_normalize_group(group)
            if group.get("fsdp_sync", False):
                raise NotImplementedError(
                    "LuminaV (MI355X build): fsdp_sync=True (sharded scratch all-reduce) is not available in this "
                    "single-GPU build."
                )
            if group.get("capturable", False):
                with torch.no_grad():
                    self._step_capturable(group, grads)
                continue
            if self._graph_steps and torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "LuminaV: a param group without capturable=True cannot be stepped inside a graph capture "
                    "(its step counts are host values a replay would repeat)."
                )
            if grads is None and not group.get("fuse_tensors", False) and self._run_unfused_plan(group):
                continue
            with torch.no_grad():
                self._step_group(group, grads)
        return loss

    def _step_group(self, group: Dict[str, Any], grads: Optional[Any]) -> None:
        """One param group: its fused buckets, or its unfused params (under no_grad)."""
        if group.get("fuse_tensors", False):
            buckets = [b for b in self._fused_buckets if b["group"] is group]
            if not buckets or any(b["buf_count"] != group["buffer"] or int(b["master_mode"]) != int(group["master_weights"])
                                  for b in buckets):
                self._sync_or_rebuild_fused_buckets()
                buckets = [b for b in self._fused_buckets if b["group"] is group]
            if buckets:
                for b in buckets:
                    self._step_bucket(group, b, grads)
                return
        self._step_unfused(group, grads)

    def _step_bucket(self, group: Dict[str, Any], b: Dict[str, Any], grads: Optional[Any]) -> None:
        """One bucket = one tensor with param_index 0 and bucket-global offsets. A slice whose
        param has no grad stays in the bucket's statistics with a zero gradient and is not
        written: it goes to the kernel as an inactive element range. The reference zeroes the grad
        slice, steps the whole bucket and copies the slice's param/state back
        (luminav.py:1426-1603); the result is the same without the copies."""
        if grads is None and self._bucket_fast_step(group, b):
            return
        flat_m, flat_v, flat_mp = b["flat_m"], b["flat_v"], b["flat_mp"]
        b["step"] = int(b["step"]) + 1
        step_t = b["step"]
        any_grad = False
        inactive: List[Tuple[int, int]] = []  # merged [begin, end) element ranges
        off = 0
        for p, p_sl, g_sl, p_ptr, g_ptr, st, idx in b["slices"]:
            n = int(p.numel())
            begin = off
            off += n
            if p.data_ptr() != p_ptr:
                p_sl.copy_(p.detach())
                p.data = p_sl
            if grads is None:
                g = p.grad
            elif isinstance(grads, (list, tuple)):
                g = grads[idx] if idx < len(grads) else None
            elif isinstance(grads, dict):
                g = grads.get(p)
            else:
                g = None
            if g is None:
                if n > 0:
                    if inactive and inactive[-1][1] == begin:
                        inactive[-1] = (inactive[-1][0], begin + n)
                    else:
                        inactive.append((begin, begin + n))
                continue
            any_grad = True
            if getattr(g, "is_sparse", False):
                b["step"] = step_t - 1
                raise RuntimeError("LuminaV does not support sparse gradients.")
            if g is not g_sl:
                validate_supported_dtype(g, "grad")
                if g.data_ptr() != g_ptr:
                    g_sl.copy_(g.detach())
                    if grads is None:
                        p.grad = g_sl
            _dict_set(st, "step", step_t)
        if not any_grad:
            b["step"] = step_t - 1
            for *_, st, _ in b["slices"]:
                st["step"] = int(st.get("step", step_t - 1))
            return
        table = None
        if inactive:
            key = tuple(inactive)
            if b.get("inactive_key") != key:  # uploaded only when the set of grad=None params changes
                b["inactive_table"] = torch.tensor(inactive, dtype=torch.int64, device=b["flat_p"].device)
                b["inactive_key"] = key
            table = b["inactive_table"]
        self._stepper.step(group, [b["flat_p"]], [b["flat_g"]], [flat_m], [flat_v], [flat_mp], [b["scratch"]],
                           [step_t], [0], inactive=[table])

    def _bucket_fast_step(self, group: Dict[str, Any], b: Dict[str, Any]) -> bool:
        """The steady bucket step: every slice's param still lives in the bucket and its grad is
        the bucket's own grad view (autograd accumulates into it), so there is no inactive range
        and nothing to copy. The checks are C-level maps over the slices and the bucket's packed
        descriptor is reused; False (nothing changed) sends the step down the general path."""
        fast = b.get("fast")
        if fast is None or fast["slices"] is not b["slices"]:
            sl = b["slices"]
            fast = b["fast"] = {
                "slices": sl, "params": [x[0] for x in sl], "g_views": [x[2] for x in sl],
                "p_ptrs": _pack_ptrs([x[3] for x in sl]), "states": [x[5] for x in sl], "prep": None,
            }
        params = fast["params"]
        if not all(map(operator.is_, map(_get_grad, params), fast["g_views"])):
            return False
        if not _same_ptrs(params, fast["p_ptrs"]):
            return False
        step_t = int(b["step"]) + 1
        prep = fast["prep"]
        if prep is None:
            prep = fast["prep"] = self._stepper.prepare([b["flat_p"]], [b["flat_g"]], [b["flat_m"]], [b["flat_v"]],
                                                        [b["flat_mp"]], [b["scratch"]], [step_t], [0])
        prep.set_steps([step_t])
        self._stepper.launch(group, prep)
        b["step"] = step_t
        any(map(_dict_set, fast["states"], repeat("step"), repeat(step_t)))
        return True

    def _step_unfused(self, group: Dict[str, Any], grads: Optional[Any]) -> None:
        """Unfused params: one C-ABI call per device over every param that has a grad
        (reference luminav.py:1932-1960 steps them one Triton launch at a time). step() has
        already tried the group's cached plan."""
        self._unfused_plans.pop(id(group), None)
        buf_count = group["buffer"]
        per_device: Dict[torch.device, List[Tuple[Any, ...]]] = {}
        plannable = grads is None
        active: List[bool] = []
        for idx, p in enumerate(group["params"]):
            g = None
            if grads is not None:
                if isinstance(grads, (list, tuple)) and idx < len(grads):
                    g = grads[idx]
                elif isinstance(grads, dict) and p in grads:
                    g = grads[p]
            if g is None:
                g = p.grad
            active.append(g is not None)
            if g is None:
                continue
            if getattr(g, "is_sparse", False):
                raise RuntimeError("LuminaV does not support sparse gradients.")
            validate_supported_dtype(p, "param")
            validate_supported_dtype(g, "grad")
            if p.numel() == 0:
                continue
            if not g.is_contiguous():
                g = g.contiguous()
                plannable = False
            if p.device.type == "cpu" and not p.is_contiguous():
                raise ValueError(
                    f"LuminaV requires parameters to be contiguous in memory for native zero-copy execution. Call .contiguous() on parameter {idx} before passing to optimizer."
                )
            p_step = p if p.is_contiguous() else p.contiguous()
            if p_step is not p:
                plannable = False
            if g.device != p.device:
                g = g.to(p.device)
                plannable = False
            state = self._init_or_refresh_state(p, group)
            state["step"] = int(state["step"]) + 1
            per_device.setdefault(p.device, []).append((
                p, p_step, g, state["exp_avg"], state.get("exp_avg_sq") if buf_count in (2, "T2") else None,
                state.get("master_param"), state["scratch"], state["step"], idx, state,
            ))
        for dev, rows in per_device.items():
            try:
                prep = self._stepper.prepare([r[1] for r in rows], [r[2] for r in rows], [r[3] for r in rows],
                                             [r[4] for r in rows], [r[5] for r in rows], [r[6] for r in rows],
                                             [r[7] for r in rows], [r[8] for r in rows])
                self._stepper.launch(group, prep)
            except ValueError:
                # rejected before anything was launched (e.g. a param listed twice: "Pointer aliasing
                # detected", as the reference's native seam raises): these params were not stepped
                for r in rows:
                    _dict_set(r[9], "step", int(r[9]["step"]) - 1)
                raise
            for r in rows:
                if r[0] is not r[1]:
                    r[0].copy_(r[1])
        if plannable and len(per_device) == 1:
            rows = next(iter(per_device.values()))
            self._unfused_plans[id(group)] = self._make_plan(group, rows, active, prep)

    def _make_plan(self, group: Dict[str, Any], rows: List[Tuple[Any, ...]], active: List[bool],
                   prep: "hip_backend.PreparedStep") -> Dict[str, Any]:
        """The cached plan of an unfused group: its packed descriptors and what a step checks
        before reusing them. Grads are held weakly (the plan must not keep last step's grads
        alive); a callback marks the plan when one of them dies, so that while none has died, equal
        object ids mean the same grad objects. The state tensors' storages are held strongly: the
        descriptors point into them, and replacing a state entry drops the plan (_ParamState), but
        nothing may free memory a plan writes."""
        dead = [False]

        def died(_ref: Any, flag: List[bool] = dead) -> None:
            flag[0] = True

        eparams = [r[0] for r in rows]
        egrads = [r[2] for r in rows]
        stensors = [t for r in rows for t in (r[3], r[4], r[5], r[6]) if t is not None]
        return {
            "epoch": self._plan_epoch, "group": group, "layout": tuple(group.get(k) for k in self._LAYOUT_KEYS),
            "params": list(group["params"]), "ids": list(map(id, group["params"])), "active": active,
            # every param has a grad and elements, so the entries follow the params one to one
            "all_active": len(rows) == len(group["params"]),
            "eparams": eparams, "pptrs": _ptr_record(eparams),
            "gids": list(map(id, egrads)), "gptrs": list(map(_data_ptr, egrads)), "gptr_rec": _ptr_record(egrads),
            "pid_rec": _pack_ptrs(list(map(id, group["params"]))),
            "gweak": [weakref.ref(g, died) for g in egrads], "dead": dead, "died": died,
            "states": [r[9] for r in rows], "steps": [int(r[7]) for r in rows], "step_epoch": self._step_epoch,
            "keep": [t.untyped_storage() for r in rows for t in (r[3], r[4], r[5], r[6]) if t is not None],
            # the state tensors themselves and where their data was: `t.data = u` or `t.set_(u)` on
            # a state tensor moves its storage without replacing the state entry
            "stensors": stensors, "sptrs": _ptr_record(stensors),
            "prep": prep,
        }

    def _run_unfused_plan(self, group: Dict[str, Any]) -> bool:
        """Steps `group` from its packed descriptors when only grads and step counters changed:
        the same params carry a grad, param and state storage is where it was and no state was
        replaced (load_state_dict, add_param_group and replacing or removing a state entry bump the epoch; a
        changed buffer count, master mode or state precision changes the recorded layout). The
        checks run as C-level maps over the whole group. Returns False, having changed nothing the
        slow path relies on, when anything else changed."""
        plan = self._unfused_plans.get(id(group))
        if plan is None or plan["epoch"] != self._plan_epoch or plan["group"] is not group:
            return False
        if plan["layout"] != tuple(map(group.get, self._LAYOUT_KEYS)):
            return False
        params = group["params"]
        prep = plan["prep"]
        # Every check in one C call (_lv_host.grad_record): the same param objects at their data
        # pointers, the state tensors at theirs, and each param's grad a dense, contiguous GPU tensor
        # of its descriptor's dtype and size. It returns where the grads are, so new grad objects
        # (zero_grad(set_to_none=True)) are taken as they come. cfg2's 64 tensors: in Python these
        # checks and the counters took 11.2 us of an 18.2 us step; with the two C calls the step is
        # 14.6 us. 2,000 tensors with new grads every step: 1.77 ms in Python.
        rec = None
        if _grad_record is not None and plan["all_active"] and type(params) is list:
            rec = _grad_record(params, plan["pid_rec"], plan["pptrs"], plan["stensors"], plan["sptrs"],
                               prep.gdtypes, prep.numels, prep.index)
        if rec is not None:
            if rec != plan["gptr_rec"]:
                prep.set_grad_record(rec)
                plan["gptr_rec"] = rec
            # the Python checks' record of the grads' identities is not kept on this path: should
            # they run, they re-point every grad
            plan["dead"][0] = True
        elif not self._check_plan_in_python(plan, params):
            return False
        # nothing above touched the step counters, so a False return leaves them for the slow path
        states = plan["states"]
        if plan["step_epoch"] != self._step_epoch:  # a counter was set from outside: read them again
            plan["steps"] = [int(st["step"]) for st in states]
            plan["step_epoch"] = self._step_epoch
        if _advance is not None:
            steps = _advance(states, plan["steps"], "step")  # also stored as each state's "step"
        else:
            steps = [s + 1 for s in plan["steps"]]
            any(map(_dict_set, states, repeat("step"), steps))  # the counters users read; None each
        plan["steps"] = steps
        prep.set_steps(steps)
        self._stepper.launch(group, prep)
        return True

    def _check_plan_in_python(self, plan: Dict[str, Any], params: List[Any]) -> bool:
        """The plan's checks one at a time: False when anything but the grads changed (the params,
        which of them have grads, where a param or state tensor's data is), else True with the
        grads that changed re-pointed (or False if one does not fit its descriptor)."""
        if list(map(id, params)) != plan["ids"]:  # the plan holds the params: equal ids, same objects
            return False
        if plan["all_active"]:
            grads = list(map(_get_grad, params))
        else:
            if [p.grad is not None for p in params] != plan["active"]:
                return False
            grads = list(map(_get_grad, plan["eparams"]))
        if not _same_ptrs(plan["eparams"], plan["pptrs"]):  # a param's storage moved
            return False
        if not _same_ptrs(plan["stensors"], plan["sptrs"]):  # a state tensor's storage moved
            return False
        gids = list(map(id, grads))
        if plan["dead"][0] or gids != plan["gids"] or not _same_ptrs(grads, plan["gptr_rec"]):
            if not self._refresh_plan_grads(plan, grads, gids):
                return False
            plan["gptr_rec"] = _ptr_record(grads)
        return True

    def _refresh_plan_grads(self, plan: Dict[str, Any], grads: List[Any], gids: List[int]) -> bool:
        """Re-points the descriptors of grads that changed (each validated: dtype, device, numel,
        contiguity, dense) and re-arms the weak references. False if a grad does not fit."""
        prep = plan["prep"]
        dead = plan["dead"]
        old_ids, old_ptrs, weak = plan["gids"], plan["gptrs"], plan["gweak"]
        if dead[0] or 4 * sum(map(operator.ne, gids, old_ids)) > len(gids):
            # the common case after zero_grad(set_to_none=True): (nearly) every grad is a new
            # tensor, so re-point them all at once (one check loop, one pointer write, weakrefs by map)
            if any(map(operator.is_, grads, repeat(None))):
                return False
            ptrs = list(map(_data_ptr, grads))
            if not prep.set_grads(grads, ptrs):
                return False
            plan["gweak"] = list(map(weakref.ref, grads, repeat(plan["died"])))
            plan["gids"] = gids
            plan["gptrs"] = ptrs
            dead[0] = False
            return True
        for k, g in enumerate(grads):
            if g is None:
                return False
            ref = weak[k]()
            if ref is g and gids[k] == old_ids[k] and g.data_ptr() == old_ptrs[k]:
                continue
            if g.is_sparse or not prep.set_grad(k, g):
                return False
            weak[k] = weakref.ref(g, plan["died"])
            old_ids[k] = gids[k]
            old_ptrs[k] = g.data_ptr()
        dead[0] = False
        return True

    # ------------------------------------------------------------------ capturable groups

    def _step_capturable(self, group: Dict[str, Any], grads: Optional[Any]) -> None:
        """capturable=True: the group's step count and its per-step coefficients live in a device
        step record (lv_step_multi_graph) that every call advances on the stream, so a HIP graph
        captured around step() (torch.cuda.graph) replays correct steps. Every parameter's
        state["step"] is then a 0-dim int64 device tensor viewing that shared count.

        The first call of a group (or the first after its parameter set or state changed) runs
        eagerly: it allocates state, the record and a workspace of the group's own, and takes a
        first step that needs the two-pass path (cautious or radial with the fused single pass)
        through lv_step_multi. Capturing a group before such a call raises. Every parameter
        stepped by the group steps together: a parameter holding state must have a grad, and one
        gaining a grad later raises (its count would start at the group's). A captured graph keeps
        the hyper-parameters (lr, betas, ...) it was captured with: capture again after changing
        them."""
        rows: List[Tuple[int, torch.Tensor, torch.Tensor]] = []
        for idx, p in enumerate(group["params"]):
            g = None
            if grads is not None:
                if isinstance(grads, (list, tuple)) and idx < len(grads):
                    g = grads[idx]
                elif isinstance(grads, dict) and p in grads:
                    g = grads[p]
            if g is None:
                g = p.grad
            if g is None:
                if p in self.state and len(self.state[p]) > 0:
                    raise ValueError(
                        f"LuminaV(capturable=True): parameter {idx} holds optimizer state but has no grad; a "
                        "capturable group steps all of its parameters together."
                    )
                continue
            if getattr(g, "is_sparse", False):
                raise RuntimeError("LuminaV does not support sparse gradients.")
            validate_supported_dtype(p, "param")
            validate_supported_dtype(g, "grad")
            if not p.is_contiguous() or not g.is_contiguous() or g.device != p.device:
                raise ValueError(
                    f"LuminaV(capturable=True): parameter {idx} and its grad must be contiguous on one device."
                )
            if p.numel() > 0:
                rows.append((idx, p, g))
        if not rows:
            return
        device = rows[0][1].device
        if any(p.device != device for _, p, _ in rows):
            raise ValueError("LuminaV(capturable=True): a capturable group's parameters share one device.")
        key = tuple(id(p) for _, p, _ in rows)
        entry = self._graph_steps.get(id(group))
        if entry is None or not self._graph_entry_valid(entry, group, key):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "LuminaV(capturable=True): take one eager step() with the same parameters before capturing a "
                    "graph; it sets up the group's state, device step record and workspace."
                )
            self._first_capturable_step(group, rows, key)
            return
        prep = entry["prep"]
        for k, (_, p, g) in enumerate(rows):
            if p.data_ptr() != entry["pptrs"][k]:
                raise RuntimeError(
                    f"LuminaV(capturable=True): the storage of parameter {rows[k][0]} moved since the group's first "
                    "step; call load_state_dict or re-create the optimizer."
                )
            if g.data_ptr() != entry["gptrs"][k]:
                if not prep.set_grad(k, g):
                    raise ValueError(f"LuminaV(capturable=True): the grad of parameter {rows[k][0]} does not fit it.")
                entry["gptrs"][k] = g.data_ptr()
        need = self._stepper.graph_workspace_bytes(group, prep)
        if need > entry["workspace"].numel():  # the options changed (e.g. to the radial bound)
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "LuminaV(capturable=True): the group's options need a larger workspace than its set-up "
                    "allocated; take one eager step() after changing them, then capture."
                )
            self._graph_retired.append(entry["workspace"])
            entry["workspace"] = self._stepper.graph_workspace(group, prep)
        self._stepper.launch_graph(group, prep, entry["record"], entry["workspace"])

    _HELD_KEYS = ("step", "exp_avg", "exp_avg_sq", "master_param", "scratch")

    def _graph_entry_valid(self, entry: Dict[str, Any], group: Dict[str, Any], key: Tuple[int, ...]) -> bool:
        """A capturable group's set-up still describes it: the same params step, its layout
        options are unchanged, and every param's state dict, counter view and state tensors are
        the objects the set-up packed (identity checks: writes to other groups' state, which drop
        the unfused plans, leave this set-up valid)."""
        if entry["group"] is not group or entry["key"] != key or entry["layout"] != tuple(map(group.get, self._LAYOUT_KEYS)):
            return False
        state = self.state
        for p, st, held in zip(entry["params"], entry["states"], entry["held"]):
            if dict.get(state, p) is not st:  # dict.get: no default entry is created
                return False
            for k, t in held:
                if dict.get(st, k) is not t:
                    return False
        # `t.data = u` or `t.set_(u)` on a state tensor moves its storage in place
        return _same_ptrs(entry["stensors"], entry["sptrs"])

    def _first_capturable_step(self, group: Dict[str, Any], rows: List[Tuple[int, torch.Tensor, torch.Tensor]],
                               key: Tuple[int, ...]) -> None:
        """Eager set-up of a capturable group (see _step_capturable)."""
        buf_count = group["buffer"]
        states = [self._init_or_refresh_state(p, group) for _, p, _ in rows]
        counts = {int(st["step"].item()) if isinstance(st["step"], torch.Tensor) else int(st["step"]) for st in states}
        if len(counts) != 1:
            raise ValueError(
                f"LuminaV(capturable=True): the group's parameters are at different steps {sorted(counts)}; a "
                "capturable group steps all of its parameters together."
            )
        done = counts.pop()
        device = rows[0][1].device
        prep = self._stepper.prepare(
            [p for _, p, _ in rows], [g for _, _, g in rows], [st["exp_avg"] for st in states],
            [st.get("exp_avg_sq") if buf_count in (2, "T2") else None for st in states],
            [st.get("master_param") for st in states], [st["scratch"] for st in states],
            [done + 1] * len(rows), [idx for idx, _, _ in rows],
        )
        record = torch.tensor([done, 0, 0, 0], dtype=torch.int64, device=device)  # lv_step_record, 32 bytes
        workspace = self._stepper.graph_workspace(group, prep)
        two_pass_first = (group["cautious"] or self._radial_active(group)) and group["fused_single_pass"]
        if done == 0 and two_pass_first:
            self._stepper.launch(group, prep)  # step 1 on the two-pass path, host step counts
            record[0] = 1
        else:
            self._stepper.launch_graph(group, prep, record, workspace)
        count = record[0]  # 0-dim view: the counter every replay advances
        for st in states:
            _dict_set(st, "step", count)
        stensors = [t for st in states for k in ("exp_avg", "exp_avg_sq", "master_param", "scratch")
                    for t in (dict.get(st, k),) if isinstance(t, torch.Tensor)]
        old = self._graph_steps.get(id(group))
        if old is not None:
            self._graph_retired += (old["record"], old["workspace"])
        self._graph_steps[id(group)] = {
            "group": group, "key": key, "layout": tuple(map(group.get, self._LAYOUT_KEYS)), "prep": prep,
            "record": record, "workspace": workspace, "params": [p for _, p, _ in rows], "states": states,
            "held": [[(k, dict.get(st, k)) for k in self._HELD_KEYS] for st in states],
            "pptrs": [p.data_ptr() for _, p, _ in rows], "gptrs": [g.data_ptr() for _, _, g in rows],
            "stensors": stensors, "sptrs": _ptr_record(stensors),
        }
