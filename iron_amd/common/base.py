"""Operator base API: the MI355X counterpart of iron/common/base.py.

The reference's operator lifecycle is kept verbatim so callers can switch
backends per operator:

    op = GEMV(M=2048, K=8192)          # dataclass; __post_init__ validates (ValueError)
    op.compile()                        # -> self
    fn = op.get_callable()              # fn(*tensors) in get_arg_spec() order
    fn(W, x, y)                         # outputs written in place

Reference: AIEOperatorBase (iron/common/base.py:33-90), MLIROperator.name
(:130-151), AIERuntimeArgSpec (:219-231).

What differs by design: there is nothing to compile per operator. All kernels
live in one prebuilt code object (libiron_hip.so, gfx950); ``compile()`` only
checks that it is loaded. Buffers are torch tensors in HBM (``cuda`` device
on ROCm), and calls are stream-ordered on torch's current stream.
"""

from __future__ import annotations

import dataclasses
import math
from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any, Callable, ClassVar

import torch

from .. import _lib
from .context import AIEContext
from .utils import float_to_name

DEVICE_NAME = "mi355x"


@dataclass(frozen=True)
class AIERuntimeArgSpec:
    """One runtime argument: direction in {"in","out","inout"}, shape, dtype.

    Mirrors iron/common/base.py:219-231; dtype is a torch dtype (bf16 default).
    """

    direction: str
    shape: tuple[int, ...]
    dtype: torch.dtype = torch.bfloat16

    def __post_init__(self) -> None:
        if self.direction not in {"in", "out", "inout"}:
            raise ValueError(
                f"Invalid direction {self.direction!r}: must be one of 'in', 'out', 'inout'"
            )

    @property
    def numel(self) -> int:
        return int(math.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * torch.empty((), dtype=self.dtype).element_size()


# Callable (operator, *cpu_tensors) -> cpu tensor behind AIEOperatorBase.reference().
_reference_provider: Callable[..., Any] | None = None


def set_reference_provider(fn: Callable[..., Any] | None) -> None:
    """Register (or clear, with None) the function that computes operators'
    CPU references, used by reference() and the compare/reference dispatch
    modes of OperatorSequence."""
    global _reference_provider
    _reference_provider = fn


def get_reference_provider() -> Callable[..., Any] | None:
    return _reference_provider


class AIEOperatorBase(ABC):
    """Base of every operator (name kept from iron/common/base.py:33)."""

    _default_context: ClassVar[AIEContext | None] = None

    def __init__(self, context: AIEContext | None = None) -> None:
        if context is None:
            context = self.get_default_context()
        self.context = context
        self._compiled = False

    @classmethod
    def get_default_context(cls) -> AIEContext:
        """Process-wide default context, created on first use (lazy singleton)."""
        if AIEOperatorBase._default_context is None:
            AIEOperatorBase._default_context = AIEContext()
        return AIEOperatorBase._default_context

    def set_up_artifacts(self) -> None:
        """Nothing to declare: every kernel is part of libiron_hip.so."""

    def compile(self, dry_run: bool = False) -> "AIEOperatorBase":
        """Load the kernel library (raises if it is not built). Returns self."""
        self.set_up_artifacts()
        if not dry_run:
            _lib.load()
        self._compiled = True
        return self

    @abstractmethod
    def get_arg_spec(self) -> list[AIERuntimeArgSpec]: ...

    @abstractmethod
    def get_callable(self) -> Callable[..., Any]: ...

    def reference(self, *inputs):
        """CPU result of this operator on CPU tensors (base.py:155-157 in the
        reference). The library ships no CPU path: the result comes from the
        provider registered with ``set_reference_provider`` (the tests register
        their CPU oracle); without one this raises."""
        if _reference_provider is None:
            raise NotImplementedError(
                f"{type(self).__name__}.reference(): no reference provider is registered; "
                "the library ships only the HIP path (register one with "
                "iron_amd.common.set_reference_provider)"
            )
        return _reference_provider(self, *inputs)

    def reference_tolerance(self):
        """Tolerance a compare-mode OperatorSequence holds this operator to
        (None: the dispatch's fallback)."""
        return None


def _serialize_param(v: object) -> str:
    if isinstance(v, bool):
        return str(int(v))
    if isinstance(v, float):
        return float_to_name(v)
    if isinstance(v, (list, tuple)):
        return "x".join(str(x) for x in v)
    return str(v)


class HIPOperator(AIEOperatorBase):
    """An operator that runs kernels of libiron_hip.so (MLIROperator's role).

    Subclasses are dataclasses that implement ``get_arg_spec`` and ``_launch``.
    ``get_callable`` validates the tensors against the arg spec and launches on
    torch's current stream of the tensors' device.
    """

    # argument index -> dtypes accepted besides the spec's own
    _extra_dtypes: ClassVar[dict] = {}
    _name_aliases: ClassVar[dict[str, str]] = {
        "num_aie_columns": "c",
        "num_channels": "ch",
        "tile_size": "t",
        "size": "sz",
        "scalar_factor": "sf",
        "rows": "r",
        "cols": "n",
    }

    @property
    def name(self) -> str:
        """Instance name from the dataclass fields (iron/common/base.py:130-151)."""
        if not dataclasses.is_dataclass(self):
            raise NotImplementedError(
                f"{type(self).__name__} must be a @dataclass or override the name property"
            )
        aliases = type(self)._name_aliases
        parts = (
            f"{aliases.get(f.name, f.name)}{_serialize_param(getattr(self, f.name))}"
            for f in dataclasses.fields(self)
            if f.repr and getattr(self, f.name) is not None
        )
        return type(self).__name__ + "_" + "_".join(parts) + "_" + DEVICE_NAME

    @abstractmethod
    def _launch(self, *args: torch.Tensor, stream: int) -> None:
        """Launch the kernel(s) on already-validated tensors."""

    def validate_args(self, args) -> None:
        specs = self.get_arg_spec()
        if len(args) != len(specs):
            raise ValueError(
                f"{type(self).__name__} takes {len(specs)} arguments, got {len(args)}"
            )
        dev = None
        for i, (t, spec) in enumerate(zip(args, specs)):
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"argument {i} of {type(self).__name__} must be a torch.Tensor")
            if t.device.type != "cuda":
                raise ValueError(
                    f"argument {i} of {type(self).__name__} must live on the GPU (got {t.device})"
                )
            if dev is None:
                dev = t.device
            elif t.device != dev:
                raise ValueError(f"argument {i} is on {t.device}, expected {dev}")
            if t.dtype != spec.dtype and t.dtype not in self._extra_dtypes.get(i, ()):
                raise ValueError(
                    f"argument {i} of {type(self).__name__} has dtype {t.dtype}, expected {spec.dtype}"
                )
            if t.numel() != spec.numel:
                raise ValueError(
                    f"argument {i} of {type(self).__name__} has {t.numel()} elements, "
                    f"expected {spec.numel} (shape {spec.shape})"
                )
            if not t.is_contiguous():
                raise ValueError(f"argument {i} of {type(self).__name__} must be contiguous")

    def get_callable(self) -> Callable[..., Any]:
        """fn(*tensors) in get_arg_spec() order. With a positive trace size (the
        operator's ``trace_size`` field, else ``IRON_TRACE_SIZE``) every call
        arms a zero-filled device buffer of that many bytes for its kernels'
        phase records (iron_trace_next_launch) and leaves it in
        ``fn.trace_buffer`` for ``tracing_utils.dump_traces`` (the reference's
        full-ELF callable and its trace buffer, iron/common/sequence.py:675-688)."""
        if not self._compiled:
            self.compile()
        _lib.load()
        from .tracing_utils import arm, new_buffer, resolve_trace_size

        trace_size = resolve_trace_size(getattr(self, "trace_size", None))

        def call(*args: torch.Tensor):
            self.validate_args(args)
            stream = _lib.stream_handle(args[0].device)
            if trace_size <= 0:
                self._launch(*args, stream=stream)
                return
            call.trace_buffer = new_buffer(trace_size, args[0].device)
            arm(call.trace_buffer)
            try:
                self._launch(*args, stream=stream)
            except BaseException:
                # a launch that failed before reaching an entry point must not
                # leave the buffer armed for a later call
                _lib.call("iron_trace_next_launch", None, 0)
                raise

        call.operator = self
        call.trace_buffer = None
        return call


# Name kept for code written against the reference (iron.common.MLIROperator).
MLIROperator = HIPOperator


class CompositeOperator(AIEOperatorBase):
    """Base class for operators that chain sub-operators (base.py:212-216)."""
