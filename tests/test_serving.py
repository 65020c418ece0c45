"""Open-loop admission and latency accounting of the serving wrapper on the
CPU, with a simulated clock and a stand-in wave loop (every wave takes 2 ms
and finishes a request after its third wave)."""
from types import SimpleNamespace

import pytest
import torch

from specgrove_amd import serving
from specgrove_amd.decode import DecodeRequest


class _Clock:
    def __init__(self):
        self.t = 0.0

    def __call__(self):
        return self.t

    def sleep(self, dt):
        self.t += dt


def _fake_loop(clock, log):
    class Loop:
        def __init__(self, model, propose, **options):
            self.device = torch.device("cpu")
            self.calls = self.rows = 0
            self.waves_of = {}

        def attach(self, states):
            for s in states:
                s.done = len(s.generated) >= 99

        def check_status(self):
            pass

        def step(self, states):
            log.append(tuple(s.request_id for s in states))
            clock.t += 0.002
            self.calls += 1
            self.rows += len(states)
            finished = []
            for s in states:
                self.waves_of[s.request_id] = self.waves_of.get(s.request_id, 0) + 1
                s.generated.append(7)
                if self.waves_of[s.request_id] == 3:
                    s.done = True
                    finished.append(s)
            return finished
    return Loop


def test_admission_respects_arrivals_and_concurrency(monkeypatch):
    clock, log = _Clock(), []
    monkeypatch.setattr(serving, "WaveLoop", _fake_loop(clock, log))
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    states = [DecodeRequest(k, [], None, None) for k in range(5)]

    def prefill(new):
        clock.t += 0.001
        for s in new:
            s.generated = [1]
            s.target_cache = object()

    res = serving.serve_open_loop(SimpleNamespace(), states, [0.0, 0.0, 0.0, 0.003, 0.05],
                                  None, prefill, max_active_requests=2, clock=clock,
                                  sleep=clock.sleep)
    assert res.max_concurrent == 2
    assert all(len(w) <= 2 for w in log)
    m = {d["request_id"]: d for d in res.request_metrics}
    # requests 0 and 1 are admitted at once; 2 waits for a free slot
    assert m[0]["admitted_ms"] == m[1]["admitted_ms"] == 0.0 and m[2]["queue_ms"] > 0
    # request 4 arrives after everything else finished: the loop sleeps until 50 ms
    assert m[4]["admitted_ms"] >= 50.0 and m[4]["queue_ms"] == pytest.approx(0.0, abs=1e-9)
    check_admissions(res, [0.0, 0.0, 0.0, 0.003, 0.05], 2)
    assert [a["admitted"] for a in res.admissions] == [(0, 1), (2, 3), (4,)]
    for d in res.request_metrics:
        assert 0 <= d["queue_ms"] <= d["ttft_ms"] <= d["e2e_ms"]
        assert d["service_ms"] == pytest.approx(d["e2e_ms"] - d["queue_ms"])
        assert d["output_tokens"] == 4
        assert d["tpot_ms"] == pytest.approx((d["completed_ms"] - d["first_token_ms"]) / 3)


def check_admissions(res, arrivals_s, max_active):
    """The admission rule of the serving decoder (serving
    continuous_tree_block_decode.py:1684-1694) on the recorded boundaries:
    everything that has arrived and is not admitted waits, and the first
    ``max_active - active`` of those in arrival order are admitted."""
    admitted_before = set()
    for entry in res.admissions:
        waiting = tuple(k for k, a in enumerate(arrivals_s)
                        if 1000 * a <= entry["at_ms"] and k not in admitted_before)
        assert entry["waiting"] == waiting
        assert entry["admitted"] == waiting[:max(0, max_active - entry["active_before"])]
        admitted_before.update(entry["admitted"])
    assert admitted_before == set(range(len(arrivals_s)))
    m = {d["request_id"]: d for d in res.request_metrics}
    for entry in res.admissions:
        for k in entry["admitted"]:
            assert m[k]["admitted_ms"] >= entry["at_ms"]


def test_contract_errors():
    states = [DecodeRequest(0, [1], None, None)]
    with pytest.raises(ValueError, match="open-loop"):
        serving.serve_open_loop(None, states, [1.0, 2.0], None, None, max_active_requests=1)
    with pytest.raises(ValueError, match="open-loop"):
        serving.serve_open_loop(None, states, [0.0], None, None, max_active_requests=0)
    with pytest.raises(ValueError, match="open-loop"):
        serving.serve_open_loop(None, states, [0.0], None, None, max_active_requests=1,
                                persistent=True)
