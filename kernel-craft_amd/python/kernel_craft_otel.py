"""
kernel_craft_otel.py
Tracing spans around kernel-craft GPU calls.

Public interface (the one kernel-craft's bridge and tests use,
``src/python/kernel_craft_otel.py`` in kernel-craft):

* ``setup_tracing(endpoint="http://localhost:4317", service_name="kernel-craft",
  exporter=None)`` installs an OpenTelemetry tracer provider once per process;
  a given exporter is attached with a synchronous processor, otherwise an OTLP
  gRPC exporter when that package is present;
* ``kernel_span(name, **attrs)`` is a context manager that opens a span named
  ``name`` carrying ``attrs`` and, when the span is recorded, sets
  ``kernel.cuda_ms`` to the device time between entering and leaving it;
* the module globals ``_tracer`` / ``_provider`` (reset to ``None`` by tests)
  and ``_get_tracer()``.

How this module decides what to do per call:

1. The span comes from the OpenTelemetry tracer when ``opentelemetry-api`` is
   importable, else from a local tracer whose spans are plain records.
2. Device timing is taken only for a span that is *recorded*: an OTEL span
   whose ``is_recording()`` is true (a provider with a sampler that keeps it),
   or a local span while a ``recorded_spans()`` block is open.  Unrecorded
   spans cost a context-manager entry and nothing on the device: no events,
   no synchronization.
3. Timing is skipped while the current stream is being captured into a graph
   (an event query there would invalidate the capture) and when no GPU is
   visible.
4. The timer records two events on the current stream and waits on the second
   one only (``Event.synchronize``), not on the whole device.
"""

from __future__ import annotations

import contextlib
import sys
import time
from typing import Any, Iterator, List, Optional

try:
    from opentelemetry import trace as _ot_trace
    _HAS_OTEL_API = True
except ImportError:
    _ot_trace = None
    _HAS_OTEL_API = False

_tracer: Any = None
_provider: Any = None

CUDA_MS_ATTR = "kernel.cuda_ms"


# ---------------------------------------------------------------------------
# Local spans: used when opentelemetry-api is not importable
# ---------------------------------------------------------------------------

class LocalSpan:
    """A finished-span record: name, attributes, wall-clock start/end (ns)."""

    context = None

    def __init__(self, name: str, recorded: bool) -> None:
        self.name = name
        self.attributes: dict = {}
        self.start_ns = time.perf_counter_ns()
        self.end_ns: Optional[int] = None
        self._recorded = recorded

    def is_recording(self) -> bool:
        return self._recorded

    def set_attribute(self, key: str, value: Any) -> None:
        self.attributes[key] = value

    def set_status(self, *args: Any, **kwargs: Any) -> None:
        pass


_sinks: List[list] = []


@contextlib.contextmanager
def recorded_spans() -> Iterator[list]:
    """Collect the local spans finished inside the block (in finishing
    order).  Only meaningful without opentelemetry-api; with it, attach an
    exporter through ``setup_tracing(exporter=...)`` instead."""
    sink: list = []
    _sinks.append(sink)
    try:
        yield sink
    finally:
        _sinks.remove(sink)


class LocalTracer:
    """Tracer of ``LocalSpan`` records; a span is recorded while some
    ``recorded_spans()`` block is open."""

    @contextlib.contextmanager
    def start_as_current_span(self, name: str, **kwargs: Any) -> Iterator[LocalSpan]:
        span = LocalSpan(name, recorded=bool(_sinks))
        try:
            yield span
        finally:
            span.end_ns = time.perf_counter_ns()
            for sink in _sinks:
                sink.append(span)


# ---------------------------------------------------------------------------
# Provider set-up
# ---------------------------------------------------------------------------

def _get_tracer() -> Any:
    """The tracer spans come from: the configured provider's, the global
    OTEL tracer (non-recording until some provider is installed), or a
    LocalTracer without opentelemetry-api."""
    global _tracer
    if _tracer is None:
        _tracer = _ot_trace.get_tracer("kernel_craft") if _HAS_OTEL_API else LocalTracer()
    return _tracer


def setup_tracing(endpoint: str = "http://localhost:4317",
                  service_name: str = "kernel-craft",
                  exporter: Any = None) -> None:
    """Install a tracer provider for kernel-craft spans (first call only;
    later calls return without change, as does any call without
    opentelemetry-api).

    ``exporter``: a SpanExporter attached through a SimpleSpanProcessor, so
    finished spans reach it before the span's ``with`` block returns.  With
    no exporter, an OTLP gRPC exporter for ``endpoint`` is attached through a
    BatchSpanProcessor if ``opentelemetry-exporter-otlp`` is importable;
    otherwise the provider records spans without exporting them."""
    global _tracer, _provider
    if not _HAS_OTEL_API or _provider is not None:
        return
    from opentelemetry.sdk.resources import Resource
    from opentelemetry.sdk.trace import TracerProvider
    from opentelemetry.sdk.trace import export as _export

    provider = TracerProvider(resource=Resource.create({"service.name": service_name}))
    if exporter is not None:
        provider.add_span_processor(_export.SimpleSpanProcessor(exporter))
    else:
        try:
            from opentelemetry.exporter.otlp.proto.grpc.trace_exporter import OTLPSpanExporter
        except ImportError:
            OTLPSpanExporter = None
        if OTLPSpanExporter is not None:
            provider.add_span_processor(
                _export.BatchSpanProcessor(OTLPSpanExporter(endpoint=endpoint, insecure=True)))
    _ot_trace.set_tracer_provider(provider)
    _provider = provider
    _tracer = provider.get_tracer("kernel_craft")


# ---------------------------------------------------------------------------
# Device timing
# ---------------------------------------------------------------------------

class _DeviceTimer:
    """A start/stop event pair on the current stream; ``None`` from
    ``begin()`` when timing is not possible or not allowed right now."""

    __slots__ = ("_torch", "_start", "_stop")

    @classmethod
    def begin(cls) -> Optional["_DeviceTimer"]:
        torch = sys.modules.get("torch")
        if torch is None:
            # The kernels take torch tensors; without torch loaded there is
            # no device work to time.
            return None
        try:
            if not torch.cuda.is_available() or torch.cuda.is_current_stream_capturing():
                return None
            t = cls()
            t._torch = torch
            t._start = torch.cuda.Event(enable_timing=True)
            t._stop = torch.cuda.Event(enable_timing=True)
            t._start.record()
            return t
        except Exception:
            return None

    def end_ms(self) -> Optional[float]:
        try:
            if self._torch.cuda.is_current_stream_capturing():
                return None
            self._stop.record()
            self._stop.synchronize()
            return float(self._start.elapsed_time(self._stop))
        except Exception:
            return None


def _recording(span: Any) -> bool:
    probe = getattr(span, "is_recording", None)
    try:
        return bool(probe()) if probe is not None else False
    except Exception:
        return False


def _set(span: Any, key: str, value: Any) -> None:
    try:
        span.set_attribute(key, value)
    except Exception:
        pass


@contextlib.contextmanager
def kernel_span(name: str, **attrs: Any) -> Iterator[Any]:
    """Span ``name`` with ``attrs`` around the block; a recorded span also
    gets ``kernel.cuda_ms``, the device time of the work the block queued on
    the current stream (events around the block, waited on at its end)."""
    with _get_tracer().start_as_current_span(name) as span:
        live = _recording(span)
        if live:
            for key, value in attrs.items():
                _set(span, key, value)
        timer = _DeviceTimer.begin() if live else None
        try:
            yield span
        finally:
            if timer is not None:
                ms = timer.end_ms()
                if ms is not None:
                    _set(span, CUDA_MS_ATTR, ms)


@contextlib.contextmanager
def null_span(name: str = "", **attrs: Any) -> Iterator[None]:
    """Drop-in for ``kernel_span`` that does nothing (same call shape)."""
    yield None
