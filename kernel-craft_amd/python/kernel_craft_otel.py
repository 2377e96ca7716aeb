"""
kernel_craft_otel.py
OpenTelemetry spans around kernel-craft GPU calls, timed with device events.

Same interface as the reference module (``src/python/kernel_craft_otel.py``):
``setup_tracing(endpoint, service_name, exporter)`` installs a tracer provider
(idempotent; a custom exporter gets a synchronous processor), and
``kernel_span(name, **attrs)`` opens a span, records a start/stop
``torch.cuda.Event`` pair on the current stream (a HIP event on ROCm) and sets
``kernel.cuda_ms`` when the span closes (reference :111-160).  Without
``opentelemetry-api`` installed, or before ``setup_tracing()``, spans are
no-ops apart from the timing.
"""

from __future__ import annotations

import contextlib
from typing import Any

try:
    from opentelemetry import trace as _ot_trace
    _HAS_OTEL_API = True
except ImportError:
    _HAS_OTEL_API = False

_tracer: Any = None
_provider: Any = None


def _get_tracer() -> Any:
    """Return the global tracer (a no-op tracer without OTEL)."""
    global _tracer
    if _tracer is None:
        _tracer = _ot_trace.get_tracer("kernel_craft") if _HAS_OTEL_API else _NoOpTracer()
    return _tracer


def setup_tracing(endpoint: str = "http://localhost:4317",
                  service_name: str = "kernel-craft",
                  exporter: Any = None) -> None:
    """Configure OpenTelemetry tracing; safe to call more than once."""
    global _tracer, _provider
    if not _HAS_OTEL_API or _provider is not None:
        return
    from opentelemetry.sdk.resources import Resource
    from opentelemetry.sdk.trace import TracerProvider
    from opentelemetry.sdk.trace.export import BatchSpanProcessor, SimpleSpanProcessor

    provider = TracerProvider(resource=Resource.create({"service.name": service_name}))
    if exporter is None:
        try:
            from opentelemetry.exporter.otlp.proto.grpc.trace_exporter import OTLPSpanExporter
            provider.add_span_processor(
                BatchSpanProcessor(OTLPSpanExporter(endpoint=endpoint, insecure=True)))
        except ImportError:
            pass
    else:
        provider.add_span_processor(SimpleSpanProcessor(exporter))
    _ot_trace.set_tracer_provider(provider)
    _provider = provider
    _tracer = provider.get_tracer("kernel_craft")


@contextlib.contextmanager
def kernel_span(name: str, **attrs: Any):
    """Span around a kernel call; sets ``kernel.cuda_ms`` from device events."""
    tracer = _get_tracer()
    start = stop = None
    try:
        import torch
        if torch.cuda.is_available():
            start = torch.cuda.Event(enable_timing=True)
            stop = torch.cuda.Event(enable_timing=True)
            start.record()
    except Exception:
        start = stop = None
    with tracer.start_as_current_span(name) as span:
        try:
            for k, v in attrs.items():
                try:
                    span.set_attribute(k, v)
                except Exception:
                    pass
            yield span
        finally:
            if start is not None and stop is not None:
                try:
                    import torch
                    stop.record()
                    torch.cuda.synchronize()
                    span.set_attribute("kernel.cuda_ms", start.elapsed_time(stop))
                except Exception:
                    pass


class _NoOpSpan:
    """Span stand-in that records attributes locally (for inspection)."""

    context = None

    def __init__(self) -> None:
        self.attributes: dict = {}

    def set_attribute(self, key: str, value: Any) -> None:
        self.attributes[key] = value

    def set_status(self, *args: Any, **kwargs: Any) -> None:
        pass


class _NoOpTracer:
    """Tracer used when opentelemetry-api is not installed."""

    @contextlib.contextmanager
    def start_as_current_span(self, name: str, **kwargs: Any):
        yield _NoOpSpan()
