"""OperatorSequence: a runlist of operators over named buffers, run as one unit.

Counterpart of iron/common/sequence.py:62-959. The API is kept:

    seq = OperatorSequence(name, runlist=[(op, "buf_a", "buf_b", "out"), ...],
                           input_args=["buf_a"], output_args=["out"],
                           buffer_sizes={"parent": nbytes}, dispatch="auto")
    seq.compile()
    fn = seq.get_callable()
    fn.get_buffer("buf_a").torch_view()[:] = x      # host view, synced before the run
    fn()                                            # runs every step, outputs synced back
    y = fn.get_buffer("out").torch_view()
    fn.params.write("name", 7); fn.params.sync()    # runtime int32 parameters

Runlist entries are ``(operator, *buffer_names)`` in the operator's arg-spec
order; a name may address a byte range of a parent buffer, ``"parent[a:b]"``
(the parent's size comes from ``buffer_sizes``). Buffers live in three arenas
(input, output, scratch) laid out as the reference lays them out
(sequence.py:408-500), with every sub-buffer aligned to 256 bytes for the
kernels' 16-byte vector loads.

Dispatch modes (sequence.py:62-300), MI355X meaning:

- ``"fused"``: the whole runlist is captured once into a hipGraph (after one
  eager warm-up run) and replayed: the counterpart of the single-ELF dispatch.
- ``"separate"``: each step is launched eagerly, one after the other.
- ``"auto"``: ``"fused"``.
- ``"compare"``: ``"separate"``, and after each step the operator's
  ``reference()`` runs on the same (device-produced) inputs; a step outside the
  tolerance is logged and, by default, raises.
- ``"reference"``: every step runs the operator's ``reference()`` on CPU
  buffers; nothing runs on the GPU.

``reference()`` implementations are not part of this library: compare and
reference modes need a provider registered with
``iron_amd.common.set_reference_provider`` (the tests register the CPU oracle).

Host/device coherence mirrors XRT buffers: each arena has a pinned host copy.
``torch_view()`` returns the host view and marks the range dirty; dirty ranges
are pushed to the GPU before a run, and the output arena is pulled back after
it. Scratch buffers are pulled on demand with ``.to("cpu")``. ``device_view()``
gives the GPU memory itself, for callers that keep data resident; ``launch()``
runs the steps without any host synchronisation.
"""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass

import torch

from .base import AIEOperatorBase, AIERuntimeArgSpec
from .graph import capture_graph

logger = logging.getLogger(__name__)

ALIGN = 256  # bytes; every sub-buffer starts on this boundary
_DEVICE_NAMES = {"npu", "gpu", "cuda", "device"}


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


# ---------------------------------------------------------------------------
# Tolerances for compare mode
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Tolerance:
    """Element-wise bound |out - ref| <= abs_tol + rel_tol * |ref|."""

    rel_tol: float
    abs_tol: float

    @classmethod
    def relative(cls, rel_tol: float, abs_tol: float = 0.0) -> "Tolerance":
        return cls(float(rel_tol), float(abs_tol))

    def check(self, out: torch.Tensor, ref: torch.Tensor) -> tuple[bool, str]:
        o = out.detach().double().reshape(-1)
        r = ref.detach().double().reshape(-1)
        bound = self.abs_tol + self.rel_tol * r.abs()
        bad = (o - r).abs() > bound
        nan_ok = torch.isnan(o) & torch.isnan(r)
        bad &= ~nan_ok
        n = int(bad.sum())
        if n == 0:
            return True, ""
        i = int(torch.nonzero(bad)[0])
        return False, f"{n}/{o.numel()} elements outside; first at {i}: {float(o[i])!r} vs {float(r[i])!r}"

    def __str__(self) -> str:
        return f"rel {self.rel_tol:g} + abs {self.abs_tol:g}"


# ---------------------------------------------------------------------------
# Dispatch policies
# ---------------------------------------------------------------------------
class SequenceDispatch:
    """How an OperatorSequence runs its steps (sequence.py:62-90)."""

    name = "base"

    def resolve(self, device) -> "SequenceDispatch":
        return self

    def set_up_artifacts(self, seq: "OperatorSequence") -> None:
        for op in seq.unique_operators():
            op.compile()

    def make_callable(self, seq: "OperatorSequence") -> "SequenceCallable":
        raise NotImplementedError


class FusedDispatch(SequenceDispatch):
    """The whole runlist as one captured hipGraph, replayed per call."""

    name = "fused"

    def make_callable(self, seq):
        return SequenceGraphCallable(seq)


class AutoDispatch(SequenceDispatch):
    """Selects ``fused`` (there is one GPU kind here)."""

    name = "auto"

    def resolve(self, device):
        return FusedDispatch()


class SeparateDispatch(SequenceDispatch):
    """Each step launched eagerly in runlist order."""

    name = "separate"

    def make_callable(self, seq):
        return SequenceEagerCallable(seq)


class CompareDispatch(SeparateDispatch):
    """``separate`` plus a per-step check against the operator's reference()
    on the same inputs (sequence.py:244-278). The GPU output propagates, so
    each comparison isolates one step."""

    name = "compare"
    FALLBACK_TOLERANCE = Tolerance.relative(0.025, 1e-2)

    def __init__(self, tolerance: Tolerance | None = None, raise_on_mismatch: bool = True):
        self.tolerance = tolerance
        self.raise_on_mismatch = raise_on_mismatch

    def step_tolerance(self, op) -> Tolerance:
        if self.tolerance is not None:
            return self.tolerance
        tol = op.reference_tolerance() if hasattr(op, "reference_tolerance") else None
        return tol if tol is not None else self.FALLBACK_TOLERANCE

    def make_callable(self, seq):
        return SequenceCompareCallable(seq, self)


class ReferenceDispatch(SequenceDispatch):
    """Every step through the operator's reference() on CPU buffers."""

    name = "reference"

    def set_up_artifacts(self, seq):
        pass

    def make_callable(self, seq):
        return SequenceReferenceCallable(seq)


_DISPATCH_ALIASES = {
    "auto": AutoDispatch,
    "fused": FusedDispatch,
    "separate": SeparateDispatch,
    "compare": CompareDispatch,
    "reference": ReferenceDispatch,
}


# ---------------------------------------------------------------------------
# The sequence
# ---------------------------------------------------------------------------
class OperatorSequence(AIEOperatorBase):
    """A runlist of operators over named buffers (sequence.py:307-547)."""

    def __init__(
        self,
        name,
        runlist,
        input_args,
        output_args,
        buffer_sizes=None,
        dispatch="auto",
        extra_flags=None,
        trace_size=0,
        share_designs=False,
        context=None,
    ):
        dispatch = self._coerce_dispatch(dispatch)
        if not all(
            isinstance(entry, tuple)
            and len(entry) >= 1
            and isinstance(entry[0], AIEOperatorBase)
            and all(isinstance(b, str) for b in entry[1:])
            for entry in runlist
        ):
            raise TypeError(
                "runlist entries must be (operator, *str) tuples; "
                "each operator must be an operator and each buffer name must be a str"
            )
        super().__init__(context=context)
        self.runlist = list(runlist)
        self.name = name + "_shared" if share_designs else name
        self.input_args = list(input_args)
        self.output_args = list(output_args)
        self.explicit_buffer_sizes = dict(buffer_sizes or {})
        self.extra_flags = list(extra_flags or [])  # accepted; nothing to pass them to
        self.trace_size = trace_size  # accepted; use rocprofv3 for traces
        self.share_designs = share_designs
        self._dispatch = dispatch

    @staticmethod
    def _coerce_dispatch(dispatch):
        if isinstance(dispatch, SequenceDispatch):
            return dispatch
        if isinstance(dispatch, str) and dispatch in _DISPATCH_ALIASES:
            return _DISPATCH_ALIASES[dispatch]()
        raise TypeError("selected dispatch mode not supported")

    @property
    def dispatch(self) -> SequenceDispatch:
        return self._dispatch

    def unique_operators(self):
        """Operators in runlist order, de-duplicated by identity."""
        seen = {}
        for op, *_ in self.runlist:
            seen.setdefault(id(op), op)
        return list(seen.values())

    def calculate_buffer_layout(self):
        """(subbuffer_layout, (input, output, scratch) sizes, slice_info).

        subbuffer_layout: name -> (arena, byte offset, byte length); slice_info:
        "parent[a:b]" -> (parent, a, b) in bytes (sequence.py:408-500).
        """
        args: dict[str, AIERuntimeArgSpec] = {}
        sliced: dict[str, tuple] = {}
        for op, *bufs in self.runlist:
            specs = op.get_arg_spec()
            if len(specs) != len(bufs):
                raise ValueError(
                    f"Number of buffers ({len(bufs)}) must match operator argument "
                    f"specification ({len(specs)}) for operator {op!r}"
                )
            for buf, spec in zip(bufs, specs):
                if "[" in buf and buf.endswith("]"):
                    base = buf[: buf.index("[")]
                    start, end = map(int, buf[buf.index("[") + 1 : -1].split(":"))
                    if base not in args and base not in self.explicit_buffer_sizes:
                        raise ValueError(
                            f"Sliced buffer '{buf}' requires explicit size for base buffer "
                            f"'{base}' in buffer_sizes parameter"
                        )
                    if end - start < spec.nbytes:
                        raise ValueError(
                            f"Sliced buffer '{buf}' holds {end - start} bytes; the operator needs {spec.nbytes}"
                        )
                    sliced[buf] = (base, start, end)
                elif buf not in args:
                    args[buf] = spec
                elif args[buf].nbytes != spec.nbytes:
                    raise ValueError(
                        f"Buffer '{buf}' has conflicting sizes between operators: "
                        f"{args[buf].shape} vs {spec.shape}"
                    )
        known = set(args) | set(sliced)
        for arg in self.input_args:
            if arg not in known and arg not in self.explicit_buffer_sizes:
                raise ValueError(f"Input argument {arg} not found in runlist buffers")
        for arg in self.output_args:
            if arg not in known and arg not in self.explicit_buffer_sizes:
                raise ValueError(f"Output argument {arg} not found in runlist buffers")

        layout: dict[str, tuple[str, int, int]] = {}

        def add(kind, names):
            offset = 0
            for a in names:
                if a in self.explicit_buffer_sizes:
                    length = int(self.explicit_buffer_sizes[a])
                elif a in args:
                    length = args[a].nbytes
                else:
                    continue
                layout[a] = (kind, offset, length)
                offset = _align(offset + length)
            return offset

        in_size = add("input", self.input_args)
        out_size = add("output", self.output_args)
        scratch = [a for a in args if a not in self.input_args and a not in self.output_args]
        scratch += [
            a for a in self.explicit_buffer_sizes
            if a not in self.input_args and a not in self.output_args and a not in scratch
        ]
        scratch_size = add("scratch", scratch)
        return layout, (in_size, out_size, scratch_size), sliced

    def set_up_artifacts(self):
        self.subbuffer_layout, self.buffer_sizes, self.slice_info = self.calculate_buffer_layout()
        self._dispatch = self._dispatch.resolve(self.context.device)
        self._dispatch.set_up_artifacts(self)

    def compile(self, dry_run: bool = False):
        self.set_up_artifacts()
        self._compiled = True
        return self

    def get_arg_spec(self):
        raise NotImplementedError(
            "OperatorSequence does not expose a unified arg spec; "
            "use get_layout_for_buffer() to inspect individual buffer layouts"
        )

    def get_callable(self):
        if not self._compiled:
            self.compile()
        return self._dispatch.make_callable(self)

    def get_layout_for_buffer(self, buffer_name):
        """(arena, offset, end) in bytes; a slice resolves to its parent's arena."""
        if buffer_name in self.slice_info:
            parent, start, end = self.slice_info[buffer_name]
            kind, p_start, _ = self.get_layout_for_buffer(parent)
            return kind, p_start + start, p_start + end
        kind, offset, length = self.subbuffer_layout[buffer_name]
        return kind, offset, offset + length


# ---------------------------------------------------------------------------
# Buffers and runtime parameters
# ---------------------------------------------------------------------------
class SequenceBuffer:
    """A named byte range of one arena (an XRT sub-buffer's role)."""

    def __init__(self, owner: "SequenceCallable", kind: str, start: int, end: int):
        self._owner, self.kind, self.start, self.end = owner, kind, start, end

    @property
    def nbytes(self) -> int:
        return self.end - self.start

    def _host_bytes(self) -> torch.Tensor:
        return self._owner._host[self.kind][self.start : self.end]

    def _device_bytes(self) -> torch.Tensor:
        return self._owner._dev[self.kind][self.start : self.end]

    def torch_view(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """Host view (bf16 by default); marks the range for upload before the next run."""
        self._owner._mark_dirty(self.kind, self.start, self.end)
        b = self._host_bytes()
        n = self.nbytes // torch.empty((), dtype=dtype).element_size()
        return b[: n * torch.empty((), dtype=dtype).element_size()].view(dtype)

    def device_view(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """The GPU memory of this buffer (no host synchronisation)."""
        b = self._device_bytes()
        size = torch.empty((), dtype=dtype).element_size()
        return b[: self.nbytes // size * size].view(dtype)

    def to(self, device: str) -> "SequenceBuffer":
        """"npu"/"gpu"/"cuda": push the host copy; "cpu": pull the device copy."""
        if self._owner._dev is None:  # reference mode: host only
            return self
        if device in _DEVICE_NAMES:
            self._device_bytes().copy_(self._host_bytes())
            self._owner._clear_dirty(self.kind, self.start, self.end)
        elif device == "cpu":
            torch.cuda.synchronize(self._owner.device)
            self._host_bytes().copy_(self._device_bytes())
        else:
            raise ValueError(f"unknown device {device!r}")
        return self

    def to_torch(self, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
        """A CPU copy of the current device contents."""
        self.to("cpu")
        size = torch.empty((), dtype=dtype).element_size()
        return self._host_bytes()[: self.nbytes // size * size].view(dtype).clone()


class SequenceParams:
    """Named int32 runtime parameters (the ParameterScratchpad's role).

    Each lives in device memory that the kernels read when they run, so a
    captured graph picks up new values on replay. ``write`` stages a value,
    ``sync`` copies the staged values to the GPU.
    """

    def __init__(self, names, device):
        self._names = list(names)
        self._index = {n: i for i, n in enumerate(self._names)}
        n = max(1, len(self._names))
        self._host = torch.zeros(n, dtype=torch.int32).pin_memory() if device is not None else torch.zeros(n, dtype=torch.int32)
        self._dev = torch.zeros(n, dtype=torch.int32, device=device) if device is not None else None

    def names(self):
        return list(self._names)

    def tensor(self, name) -> torch.Tensor:
        """The one-element device tensor holding parameter ``name``."""
        i = self._index[name]
        return self._dev[i : i + 1] if self._dev is not None else self._host[i : i + 1]

    def write(self, name, value) -> None:
        if name not in self._index:
            raise KeyError(f"unknown runtime parameter {name!r} (known: {self._names})")
        self._host[self._index[name]] = int(value)

    def read(self, name) -> int:
        return int(self._host[self._index[name]])

    def sync(self) -> None:
        if self._dev is not None:
            self._dev.copy_(self._host)


def _runtime_parameters(op):
    """(parameter name, setter) pairs an operator reads from device memory."""
    out = []
    name = getattr(op, "vector_size_parameter", None)
    if name:
        out.append((name, lambda t, op=op: setattr(op, "_vector_size_dev", t)))
    name = getattr(op, "position_parameter", None)
    if name:
        out.append((name, lambda t, op=op: setattr(op, "position_tensor", t)))
    name = getattr(op, "input_offset_parameter", None)
    if name:
        out.append((name, lambda t, op=op: setattr(op, "_in_addend_dev", t)))
    name = getattr(op, "output_offset_parameter", None)
    if name:
        out.append((name, lambda t, op=op: setattr(op, "_out_addend_dev", t)))
    return out


# ---------------------------------------------------------------------------
# Callables
# ---------------------------------------------------------------------------
class SequenceCallable:
    """Runs an OperatorSequence; ``get_buffer`` hands out named buffers."""

    uses_device = True

    def __init__(self, op: OperatorSequence):
        self.op = op
        self.last_elapsed = 0.0
        self.device = op.context.device if self.uses_device else None
        self._buffer_cache: dict[str, SequenceBuffer] = {}
        self._dirty: dict[str, list[tuple[int, int]]] = {"input": [], "output": [], "scratch": []}
        sizes = dict(zip(("input", "output", "scratch"), op.buffer_sizes))
        pin = self.uses_device
        self._host = {k: torch.zeros(max(v, ALIGN), dtype=torch.uint8) for k, v in sizes.items()}
        if pin:
            self._host = {k: t.pin_memory() for k, t in self._host.items()}
        self._dev = (
            {k: torch.zeros(max(v, ALIGN), dtype=torch.uint8, device=self.device) for k, v in sizes.items()}
            if self.uses_device
            else None
        )
        params = []
        for step_op in op.unique_operators():
            params += _runtime_parameters(step_op)
        self.params = SequenceParams(dict.fromkeys(n for n, _ in params), self.device)
        for name, setter in params:
            setter(self.params.tensor(name))

    # --- buffers -----------------------------------------------------------
    def get_buffer(self, buffer_name) -> SequenceBuffer:
        buf = self._buffer_cache.get(buffer_name)
        if buf is None:
            if buffer_name not in self.op.subbuffer_layout and buffer_name not in self.op.slice_info:
                raise ValueError(f"Unknown buffer '{buffer_name}' in runlist")
            kind, start, end = self.op.get_layout_for_buffer(buffer_name)
            buf = SequenceBuffer(self, kind, start, end)
            self._buffer_cache[buffer_name] = buf
        return buf

    def _mark_dirty(self, kind, start, end):
        self._dirty[kind].append((start, end))

    def _clear_dirty(self, kind, start, end):
        self._dirty[kind] = [(a, b) for a, b in self._dirty[kind] if a < start or b > end]

    def _arg_tensor(self, name: str, spec: AIERuntimeArgSpec, host: bool = False) -> torch.Tensor:
        kind, start, _ = self.op.get_layout_for_buffer(name)
        arena = self._host[kind] if host else self._dev[kind]
        return arena[start : start + spec.nbytes].view(spec.dtype).view(spec.shape)

    def _steps(self):
        """(operator, [(name, spec), ...]) per runlist step."""
        for step_op, *names in self.op.runlist:
            specs = step_op.get_arg_spec()
            if len(specs) != len(names):
                raise ValueError(
                    f"Operator {step_op!r} arg-spec count {len(specs)} does not match runlist buffer count {len(names)}"
                )
            yield step_op, list(zip(names, specs))

    # --- synchronisation ---------------------------------------------------
    def _sync_inputs(self):
        for kind, ranges in self._dirty.items():
            for a, b in ranges:
                self._dev[kind][a:b].copy_(self._host[kind][a:b], non_blocking=True)
            ranges.clear()
        self.params.sync()

    def _sync_outputs(self):
        torch.cuda.synchronize(self.device)
        self._host["output"].copy_(self._dev["output"])

    # --- running -----------------------------------------------------------
    def _run(self):
        raise NotImplementedError

    def launch(self):
        """Run every step on the current stream; no host synchronisation."""
        self._run()

    def __call__(self):
        with torch.cuda.device(self.device):
            self._sync_inputs()
            t0 = time.perf_counter()
            self._run()
            torch.cuda.synchronize(self.device)
            self.last_elapsed = time.perf_counter() - t0
            self._sync_outputs()


class SequenceEagerCallable(SequenceCallable):
    """Each step launched in order on the current stream."""

    def _run(self):
        for step_op, args in self._steps():
            step_op.get_callable()(*(self._arg_tensor(n, s) for n, s in args))


class SequenceGraphCallable(SequenceEagerCallable):
    """The runlist captured once into a hipGraph and replayed."""

    def __init__(self, op):
        super().__init__(op)
        self._graph = None

    def _capture(self):
        # one eager run first: operators allocate their own scratch on first use
        SequenceEagerCallable._run(self)
        self._graph = capture_graph(lambda: SequenceEagerCallable._run(self), self.device)

    def _run(self):
        if self._graph is None:
            self._capture()  # the warm-up run already produced this call's results
            return
        self._graph.replay()


class SequenceCompareCallable(SequenceEagerCallable):
    """Eager steps, each checked against its operator's reference() on the
    same device-produced inputs (sequence.py:905-959)."""

    def __init__(self, op, dispatch: CompareDispatch):
        super().__init__(op)
        self.dispatch = dispatch
        self.raise_on_mismatch = dispatch.raise_on_mismatch
        self.last_step_stats: list[dict] = []

    def _run(self):
        self.last_step_stats = []
        for idx, (step_op, args) in enumerate(self._steps()):
            tensors = [self._arg_tensor(n, s) for n, s in args]
            torch.cuda.synchronize(self.device)
            *in_args, (out_name, out_spec) = args
            cpu_inputs = [t.detach().cpu().clone() for t in tensors[:-1]]
            step_op.get_callable()(*tensors)
            torch.cuda.synchronize(self.device)
            out = tensors[-1].detach().cpu()
            ref = step_op.reference(*cpu_inputs).reshape(out_spec.shape)
            diff = (out.double() - ref.double()).abs()
            stats = {
                "step": idx,
                "op": type(step_op).__name__,
                "op_name": getattr(step_op, "name", type(step_op).__name__),
                "inputs": [n for n, _ in in_args],
                "output": out_name,
                "max_abs": float(diff.max()) if diff.numel() else 0.0,
                "mean_abs": float(diff.mean()) if diff.numel() else 0.0,
                "ref_max": float(ref.double().abs().max()) if ref.numel() else 0.0,
            }
            tol = self.dispatch.step_tolerance(step_op)
            ok, detail = tol.check(out, ref)
            stats["mismatch"] = not ok
            self.last_step_stats.append(stats)
            logger.log(
                logging.INFO if ok else logging.ERROR,
                "[compare step %d] %s -> %s: max_abs=%.4g mean_abs=%.4g ref_max=%.4g%s",
                idx, stats["op"], out_name, stats["max_abs"], stats["mean_abs"], stats["ref_max"],
                "" if ok else f"  MISMATCH: {detail}",
            )
            if not ok and self.raise_on_mismatch:
                raise RuntimeError(
                    f"[compare step {idx}] {stats['op']} (name={stats['op_name']}) -> {out_name}: "
                    f"GPU output deviates from reference ({detail}; tolerance {tol})"
                )


class SequenceReferenceCallable(SequenceCallable):
    """CPU-only evaluation through each operator's reference(); no GPU."""

    uses_device = False

    def _sync_inputs(self):
        for ranges in self._dirty.values():
            ranges.clear()

    def _sync_outputs(self):
        pass

    def _run(self):
        for step_op, args in self._steps():
            *in_args, (out_name, out_spec) = args
            inputs = [self._arg_tensor(n, s, host=True).clone() for n, s in in_args]
            out = step_op.reference(*inputs)
            dst = self._arg_tensor(out_name, out_spec, host=True)
            dst.copy_(out.reshape(out_spec.shape).to(out_spec.dtype))

    def __call__(self):
        t0 = time.perf_counter()
        self._run()
        self.last_elapsed = time.perf_counter() - t0
