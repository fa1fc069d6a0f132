"""Scan metrics and routing traces of a decode step on the GPU.

``ScanMetrics`` restates components/stream/crates/spm-stream-metrics
(model.rs:9-40, rates.rs:5-63, ratios.rs:5-33): raw counters of one pass over
the parameters and the ratios derived from them, each None when its
denominator is zero.  ``RouteEvent`` / ``RoutingTrace`` and ``ExpertEvent`` /
``Trace`` restate the JSON schemas of components/cli/crates/spm-viz-trace/
src/lib.rs:1-133 (schema names, field order, event bounds, refusals).

The counters come from the device here, not from a file scan:

* parameter_bytes_read -- the algorithmic weight bytes of the step: every
  weight row the step reads, once (all matrices of a dense model; attention,
  router, shared FFN, the distinct routed experts and the output rows of a
  mixture-of-experts model, the experts taken from the device route trace);
* weights_decoded -- the weights those bytes hold;
* weight_applications -- each weight times the tokens it is applied to
  (every client for the shared matrices, the tokens routed to it for an
  expert), so Ps is the reuse that batching and expert sharing buy;
* resident_parameter_bytes / total_parameter_bytes -- parameter bytes held
  in HBM over the model's (1 for a resident model, less with the expert
  cache);
* storage_time -- the time the store needs to deliver parameter_bytes_read
  at the rate measured on the same device (emu_hbm_read_rate: a read-only
  stream of a buffer larger than the Infinity Cache), so raw_bandwidth is
  that measured rate; absent a measured rate, storage_time is 0 and
  raw_bandwidth and eta are None (nothing is assumed);
* compute_time -- the measured step;
* wall_time -- the measured step as well: on the GPU the HBM stream and the
  arithmetic run inside the same kernels, overlapped, which is the case the
  reference's elapsed() anticipates (model.rs:31-40: with overlap the sum
  becomes an upper bound), so elapsed() is the measured wall clock and the
  weight rates are over it.  eta = storage / compute is the step's fraction
  of the measured HBM rate: eta < 1 says the engine, not HBM, sets the pace.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from .gguf import row_bytes

HBM_PEAK_BYTES_PER_S = 8.0e12  # published peak: for roofline fractions only, never a storage time


def widen(value: int) -> float:
    """u64 -> f64 through its two 32-bit halves (model.rs:56-60)."""
    high, low = (value >> 32) & 0xFFFFFFFF, value & 0xFFFFFFFF
    return float(high) * 4294967296.0 + float(low)


@dataclass
class ScanMetrics:
    parameter_bytes_read: int = 0
    weights_decoded: int = 0
    weight_applications: int = 0
    resident_parameter_bytes: int = 0
    total_parameter_bytes: int = 0
    storage_time: float = 0.0  # seconds
    compute_time: float = 0.0  # seconds
    wall_time: Optional[float] = None  # seconds, when storage and compute overlap

    def elapsed(self) -> float:
        """Storage + compute when they do not overlap (model.rs:31-40); the
        measured wall clock when they do."""
        return self.wall_time if self.wall_time is not None else self.storage_time + self.compute_time

    def scan_productivity(self) -> Optional[float]:
        """Ps: useful parameter applications per weight read."""
        return widen(self.weight_applications) / widen(self.weights_decoded) if self.weights_decoded > 0 else None

    def residency(self) -> Optional[float]:
        """Rp: parameter bytes resident over the model's parameter bytes."""
        if self.total_parameter_bytes == 0:
            return None
        return widen(self.resident_parameter_bytes) / widen(self.total_parameter_bytes)

    def raw_bandwidth(self) -> Optional[float]:
        return widen(self.parameter_bytes_read) / self.storage_time if self.storage_time > 0 else None

    def decoded_weights_per_sec(self) -> Optional[float]:
        s = self.elapsed()
        return widen(self.weights_decoded) / s if s > 0 else None

    def useful_weights_per_sec(self) -> Optional[float]:
        s = self.elapsed()
        return widen(self.weight_applications) / s if s > 0 else None

    def eta(self) -> Optional[float]:
        return self.storage_time / self.compute_time if self.compute_time > 0 else None

    def report(self) -> dict:
        r = lambda v: None if v is None else round(v, 6)  # noqa: E731
        return {"Ps": r(self.scan_productivity()), "Rp": r(self.residency()), "eta": r(self.eta()),
                "raw_bandwidth_bytes_per_s": r(self.raw_bandwidth()),
                "decoded_weights_per_s": r(self.decoded_weights_per_sec()),
                "useful_weights_per_s": r(self.useful_weights_per_sec()),
                "parameter_bytes_read": self.parameter_bytes_read, "weights_decoded": self.weights_decoded,
                "weight_applications": self.weight_applications,
                "resident_parameter_bytes": self.resident_parameter_bytes,
                "total_parameter_bytes": self.total_parameter_bytes,
                "storage_time_s": r(self.storage_time), "compute_time_s": r(self.compute_time),
                "elapsed_s": r(self.elapsed())}


# ---- traces (spm-viz-trace/src/lib.rs) ------------------------------------

@dataclass
class RouteEvent:
    layer: int
    token: int
    experts: list


@dataclass
class RoutingTrace:
    """Schema emufpga.moe-routing.v1 (lib.rs:25-80) when the model routes 8
    of at most 32 experts, as v1 requires (ids below 32, exactly 8 per
    event).  Wider models (OLMoE's 64, the Gemma-4 form's 128 experts, or
    another k) write emufpga-amd.moe-routing.wide.v1: the same fields and
    event bound, ids below n_experts (at most 256), k experts per event."""
    model: str
    events: list = field(default_factory=list)
    n_experts: int = 32
    k: int = 8
    MAX_EVENTS = 24 * 128

    @property
    def schema(self) -> str:
        return "emufpga.moe-routing.v1" if self.n_experts <= 32 and self.k == 8 else "emufpga-amd.moe-routing.wide.v1"

    def push(self, event: RouteEvent) -> None:
        """Refuses past the event bound, out-of-range ids and events of
        another width (lib.rs:41-56)."""
        if len(self.events) == self.MAX_EVENTS:
            raise ValueError(f"routing trace exceeds {self.MAX_EVENTS:,} events")
        bound = 32 if self.schema == "emufpga.moe-routing.v1" else min(self.n_experts, 256)
        if any(e >= bound or e < 0 for e in event.experts):
            raise ValueError(f"routing trace expert is outside 0..{bound}")
        if len(event.experts) != self.k:
            raise ValueError(f"routing trace event holds {len(event.experts)} experts, not {self.k}")
        if not (0 <= event.layer < 256 and 0 <= event.token < 65536):
            raise ValueError("routing trace layer or token out of range")
        self.events.append(event)

    def to_json(self) -> str:
        ev = ",".join('{"layer":%d,"token":%d,"experts":[%s]}' % (e.layer, e.token, ",".join(str(int(x))
                                                                                            for x in e.experts))
                      for e in self.events)
        return '{"schema":"%s","model":"%s","events":[%s]}' % (self.schema, self.model, ev)


@dataclass
class ExpertEvent:
    layer: int
    expert: int
    selected: bool
    routed_tokens: int
    packed_bytes: int
    decoded_bytes: int
    layer_read_us: int
    layer_decode_us: int
    layer_compute_us: int

    def to_json(self) -> str:
        return ('{"layer":%d,"expert":%d,"selected":%s,"routed_tokens":%d,"packed_bytes":%d,"decoded_bytes":%d,'
                '"layer_read_us":%d,"layer_decode_us":%d,"layer_compute_us":%d}'
                % (self.layer, self.expert, "true" if self.selected else "false", self.routed_tokens,
                   self.packed_bytes, self.decoded_bytes, self.layer_read_us, self.layer_decode_us,
                   self.layer_compute_us))


@dataclass
class Trace:
    model: str
    schedule: str
    events: list = field(default_factory=list)
    MAX_EVENTS = 24 * 32

    def push(self, event: ExpertEvent) -> None:
        if len(self.events) == self.MAX_EVENTS:
            raise ValueError(f"visualization trace exceeds {self.MAX_EVENTS} events")
        self.events.append(event)

    def to_json(self) -> str:
        return ('{"schema":"emufpga.serial-moe.v1","model":"%s","schedule":"%s",'
                '"timing_scope":"measured-layer-total","events":[%s]}'
                % (self.model, self.schedule, ",".join(e.to_json() for e in self.events)))


def next_frame(current: int, event_count: int, playing: bool) -> int:
    """lib.rs:126-133."""
    return (current + 1) % event_count if playing and event_count > 0 else current


# ---- filled from the device ----------------------------------------------

def _weights(cols_rows_enc) -> tuple[int, int]:
    """(bytes, weights) of matrices given as (rows, cols, encoding)."""
    b = w = 0
    for rows, cols, enc in cols_rows_enc:
        b += rows * row_bytes(enc, cols)
        w += rows * cols
    return b, w


def _shared_matrices(cfg) -> list:
    """(rows, cols, encoding) of every matrix each token of a step reads:
    the dense layers, or the MoE layers' attention, f32 router and shared
    FFN; then the output rows."""
    H, QW, KW = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    enc = cfg.encoding
    per = [(QW + 2 * KW, H, enc), (H, QW, enc)]
    if cfg.n_experts:
        per.append((cfg.n_experts, H, 0))  # f32 router
        if cfg.gemma and cfg.shared_ff:
            per += [(2 * cfg.shared_ff, H, enc), (H, cfg.shared_ff, enc)]
    else:
        per += [(2 * cfg.ffn, H, enc), (H, cfg.ffn, enc)]
    return per * cfg.layers + [(cfg.vocab, H, enc)]


def _expert_matrices(cfg) -> list:
    down = cfg.expert_down_encoding if cfg.gemma else cfg.expert_encoding
    return [(2 * cfg.expert_ff, cfg.hidden, cfg.expert_encoding), (cfg.hidden, cfg.expert_ff, down)]


def model_parameter_bytes(cfg) -> int:
    """Parameter bytes of the model: every matrix (experts included), the
    embedding when it is not the output, and the f32 gains."""
    b, _ = _weights(_shared_matrices(cfg))
    if cfg.n_experts:
        eb, _ = _weights(_expert_matrices(cfg))
        b += cfg.layers * cfg.n_experts * eb
    if not cfg.tied:
        b += cfg.vocab * row_bytes(cfg.encoding, cfg.hidden)
    gains = 2 * cfg.layers * cfg.hidden + 2 * cfg.layers * cfg.head_dim + cfg.hidden
    return b + 4 * gains


def step_metrics(cfg, n_clients: int, step_seconds: float, routes: Optional[np.ndarray] = None,
                 resident_bytes: Optional[int] = None, hbm_bytes_per_s: Optional[float] = None,
                 read_bytes: Optional[int] = None) -> ScanMetrics:
    """ScanMetrics of one decode step of n_clients.  routes: the step's expert
    ids [layer][client][k] from the device route trace (MoE models);
    hbm_bytes_per_s: the HBM read rate measured on the device
    (emu_hbm_read_rate), which sets storage_time (0 without it); read_bytes:
    the step's HBM bytes as a counter pass measured them (FETCH_SIZE), in
    place of the algorithmic bytes."""
    sb, sw = _weights(_shared_matrices(cfg))
    read_b, read_w, apps = sb, sw, sw * n_clients
    if cfg.n_experts:
        if routes is None:
            raise ValueError("a mixture-of-experts step needs its routes")
        eb, ew = _weights(_expert_matrices(cfg))
        for layer in range(cfg.layers):
            ids, counts = np.unique(np.asarray(routes[layer]).reshape(-1), return_counts=True)
            read_b += eb * ids.size
            read_w += ew * ids.size
            apps += ew * int(counts.sum())
    total = model_parameter_bytes(cfg)
    if read_bytes is not None:
        read_b = read_bytes
    return ScanMetrics(parameter_bytes_read=int(read_b), weights_decoded=int(read_w), weight_applications=int(apps),
                       resident_parameter_bytes=int(total if resident_bytes is None else resident_bytes),
                       total_parameter_bytes=int(total),
                       storage_time=read_b / hbm_bytes_per_s if hbm_bytes_per_s else 0.0,
                       compute_time=step_seconds, wall_time=step_seconds)


def routing_trace(model: str, steps_routes, n_clients: int, n_experts: int, max_events: Optional[int] = None
                  ) -> RoutingTrace:
    """RouteEvents of traced steps (each [layer][client][k] ids): token =
    step * n_clients + client, as many events as the schema's bound allows."""
    k = int(np.asarray(steps_routes[0]).shape[-1]) if len(steps_routes) else 8
    t = RoutingTrace(model=model, n_experts=n_experts, k=k)
    limit = t.MAX_EVENTS if max_events is None else min(max_events, t.MAX_EVENTS)
    for s, ids in enumerate(steps_routes):
        for layer in range(ids.shape[0]):
            for c in range(n_clients):
                if len(t.events) == limit:
                    return t
                t.push(RouteEvent(layer=layer, token=s * n_clients + c, experts=[int(x) for x in ids[layer, c]]))
    return t


def expert_trace(model: str, cfg, routes: np.ndarray, layer_us, layers: Optional[int] = None) -> Trace:
    """ExpertEvents of one traced step: every (layer, expert) with whether the
    step routed to it and how many tokens, its packed bytes and decoded
    (f32) bytes, and the layer's measured time (layer_us[layer], from
    emu_session_time_layers: HIP events around each layer's kernels).  The
    GPU streams and decodes inside the same kernels as the arithmetic, so
    there is no separate read or decode phase: those times are 0 and the
    whole layer interval is compute."""
    t = Trace(model=model, schedule="gpu-resident")
    eb, ew = _weights(_expert_matrices(cfg))
    for layer in range(cfg.layers if layers is None else min(layers, cfg.layers)):
        us = int(round(float(layer_us[layer])))
        ids = np.asarray(routes[layer]).reshape(-1)
        for e in range(cfg.n_experts):
            n = int(np.count_nonzero(ids == e))
            if len(t.events) == t.MAX_EVENTS:
                return t
            t.push(ExpertEvent(layer=layer, expert=e, selected=n > 0, routed_tokens=n, packed_bytes=eb,
                               decoded_bytes=4 * ew, layer_read_us=0, layer_decode_us=0, layer_compute_us=us))
    return t


__all__ = ["ScanMetrics", "widen", "RouteEvent", "RoutingTrace", "ExpertEvent", "Trace", "next_frame",
           "step_metrics", "model_parameter_bytes", "routing_trace", "expert_trace"]
