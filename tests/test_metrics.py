"""Scan metrics and traces (CPU only): the reference's known answers
(components/stream/crates/spm-stream-metrics/tests/known_answers.rs,
rates_and_edges.rs; components/cli/crates/spm-viz-trace/tests/schema.rs) and
the accounting of a GPU decode step."""
import json

import numpy as np
import pytest

from emufpga_amd import metrics as M
from emufpga_amd.gguf import row_bytes
from emufpga_amd.serve import GRANITE_MOE_Q6K, OLMOE_1B_7B, QWEN3_8B_Q6K


def batch_one():  # known_answers.rs:11-21
    return M.ScanMetrics(parameter_bytes_read=1000, weights_decoded=4000, weight_applications=4000,
                         resident_parameter_bytes=16, total_parameter_bytes=1000, storage_time=2.0, compute_time=1.0)


def test_known_answers():
    b = batch_one()
    assert b.scan_productivity() == 1.0                                   # known_answers.rs:24-30
    b32 = M.ScanMetrics(**{**b.__dict__, "weight_applications": 4000 * 32})
    assert b32.scan_productivity() == 32.0 and b32.raw_bandwidth() == b.raw_bandwidth()  # :32-46
    assert b.residency() == 0.016                                        # :48-60
    assert M.ScanMetrics(**{**b.__dict__, "resident_parameter_bytes": 1000}).residency() == 1.0
    assert b.eta() == 2.0                                                 # :62-78
    assert M.ScanMetrics(**{**b.__dict__, "storage_time": 1.0, "compute_time": 4.0}).eta() == 0.25


def test_rates_and_edges():
    m = M.ScanMetrics(parameter_bytes_read=1000, storage_time=2.0, compute_time=8.0)
    assert m.raw_bandwidth() == 500.0                                     # rates_and_edges.rs:7-19
    m = M.ScanMetrics(weights_decoded=4000, weight_applications=32000, storage_time=2.0, compute_time=2.0)
    assert m.elapsed() == 4.0 and m.decoded_weights_per_sec() == 1000.0 and m.useful_weights_per_sec() == 8000.0
    e = M.ScanMetrics()                                                   # :37-49
    assert (e.scan_productivity(), e.residency(), e.eta(), e.raw_bandwidth(), e.decoded_weights_per_sec()) == \
        (None,) * 5
    big = M.ScanMetrics(parameter_bytes_read=1 << 40, weights_decoded=1 << 40, weight_applications=1 << 42,
                        storage_time=1.0, compute_time=1.0)
    assert big.raw_bandwidth() == 1_099_511_627_776.0 and big.scan_productivity() == 4.0  # :51-64
    assert M.widen((1 << 53) + 2) == float((1 << 53) + 2)


def test_trace_schemas():  # spm-viz-trace/tests/schema.rs
    ev = M.ExpertEvent(layer=2, expert=7, selected=True, routed_tokens=3, packed_bytes=1_314_816,
                       decoded_bytes=6_291_456, layer_read_us=14_000, layer_decode_us=9_000, layer_compute_us=60_000)
    t = M.Trace(model="granite-test", schedule="all-expert")
    t.push(ev)
    js = t.to_json()
    for f in ['emufpga.serial-moe.v1', 'measured-layer-total', '"layer":2', '"expert":7', '"selected":true',
              '"routed_tokens":3', '"packed_bytes":1314816', '"decoded_bytes":6291456', '"layer_read_us":14000',
              '"layer_decode_us":9000', '"layer_compute_us":60000']:
        assert f in js
    json.loads(js)
    t = M.Trace(model="granite-test", schedule="all-expert")
    for _ in range(M.Trace.MAX_EVENTS):
        t.push(ev)
    with pytest.raises(ValueError):
        t.push(ev)
    assert (M.next_frame(3, 8, False), M.next_frame(3, 8, True), M.next_frame(7, 8, True),
            M.next_frame(0, 0, True)) == (3, 4, 0, 0)
    r = M.RoutingTrace(model="granite-test")
    r.push(M.RouteEvent(layer=2, token=7, experts=[1, 3, 5, 7, 9, 11, 13, 15]))
    assert r.to_json() == ('{"schema":"emufpga.moe-routing.v1","model":"granite-test","events":[{"layer":2,'
                           '"token":7,"experts":[1,3,5,7,9,11,13,15]}]}')
    with pytest.raises(ValueError):
        r.push(M.RouteEvent(layer=0, token=0, experts=[32, 0, 1, 2, 3, 4, 5, 6]))
    with pytest.raises(ValueError):  # v1 holds exactly 8 experts per event
        r.push(M.RouteEvent(layer=0, token=0, experts=[1, 2, 3]))
    # wider models keep v1's fields under their own schema name and bounds
    w = M.RoutingTrace(model="olmoe-test", n_experts=64)
    w.push(M.RouteEvent(layer=1, token=3, experts=[63, 40, 32, 0, 1, 2, 3, 4]))
    assert json.loads(w.to_json())["schema"] == "emufpga-amd.moe-routing.wide.v1"
    with pytest.raises(ValueError):
        w.push(M.RouteEvent(layer=0, token=0, experts=[64, 0, 1, 2, 3, 4, 5, 6]))
    assert M.RoutingTrace(model="k2", n_experts=16, k=2).schema == "emufpga-amd.moe-routing.wide.v1"


def test_dense_step_accounting():
    cfg = QWEN3_8B_Q6K
    m = M.step_metrics(cfg, 8, 3.3e-3, hbm_bytes_per_s=6.1e12)
    assert m.parameter_bytes_read == 6_208_204_800  # every weight row once, the output rows included
    assert m.scan_productivity() == 8.0 and m.residency() == 1.0
    # storage time at the measured rate; raw bandwidth is that rate back
    assert abs(m.eta() - 6_208_204_800 / 6.1e12 / 3.3e-3) < 1e-12
    assert abs(m.raw_bandwidth() - 6.1e12) < 1.0
    # storage overlaps compute on the GPU: the rates are over the measured step
    assert m.elapsed() == 3.3e-3
    assert abs(m.decoded_weights_per_sec() - m.weights_decoded / 3.3e-3) < 1e-3
    # no measured rate: nothing is assumed
    u = M.step_metrics(cfg, 1, 1.8e-3)
    assert u.storage_time == 0.0 and u.raw_bandwidth() is None and u.eta() == 0.0
    # without overlap (no wall time) the reference's sum
    s = M.ScanMetrics(parameter_bytes_read=10, weights_decoded=10, weight_applications=10, storage_time=1.0,
                      compute_time=2.0)
    assert s.elapsed() == 3.0


def test_moe_step_accounting_counts_distinct_experts_and_routed_tokens():
    cfg = GRANITE_MOE_Q6K
    rng = np.random.default_rng(0)
    routes = np.stack([np.stack([rng.choice(32, 8, replace=False) for _ in range(4)]) for _ in range(cfg.layers)])
    m = M.step_metrics(cfg, 4, 1.5e-3, routes)
    per_expert = 2 * 512 * row_bytes(14, 1024) + 1024 * row_bytes(14, 512)
    distinct = sum(len(set(routes[l].reshape(-1).tolist())) for l in range(cfg.layers))
    shared = cfg.layers * ((1024 + 2 * 512) * row_bytes(14, 1024) + 1024 * row_bytes(14, 1024) + 4 * 32 * 1024) \
        + cfg.vocab * row_bytes(14, 1024)
    assert m.parameter_bytes_read == shared + distinct * per_expert
    # every token applies each of its 8 experts' weights once
    apps = 4 * (m.weights_decoded - distinct * 3 * 512 * 1024) + cfg.layers * 4 * 8 * 3 * 512 * 1024
    assert m.weight_applications == apps
    assert 1.0 < m.scan_productivity() < 4.0
    tr = M.routing_trace("granite", [routes, routes], 4, 32)
    assert len(tr.events) == 2 * cfg.layers * 4 and tr.events[-1].token == 7
    layer_us = [50.0 + l for l in range(cfg.layers)]
    et = M.expert_trace("granite", cfg, routes, layer_us)
    assert len(et.events) == cfg.layers * 32
    assert [et.events[32 * l].layer_compute_us for l in range(cfg.layers)] == [50 + l for l in range(cfg.layers)]
    assert sum(e.routed_tokens for e in et.events) == cfg.layers * 4 * 8
    with pytest.raises(ValueError):
        M.step_metrics(OLMOE_1B_7B, 8, 1e-3)  # an MoE step needs its routes


def test_measured_read_bytes_replace_the_algorithmic_ones():
    cfg = QWEN3_8B_Q6K
    m = M.step_metrics(cfg, 1, 1.8e-3, hbm_bytes_per_s=5.9e12, read_bytes=6_284_260_277)
    assert m.parameter_bytes_read == 6_284_260_277
    assert abs(m.storage_time - 6_284_260_277 / 5.9e12) < 1e-15
    assert m.weights_decoded == M.step_metrics(cfg, 1, 1.8e-3).weights_decoded
