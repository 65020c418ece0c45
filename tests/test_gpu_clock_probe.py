"""The measurement probe bench.py brackets its timed windows with: per-XCD
shader clock from the shader-cycle and wall-clock counters of each CU."""
import pytest
import torch

from specgrove_amd import ops

pytestmark = pytest.mark.gpu


def test_clock_probe_reads_a_plausible_clock_on_every_xcd():
    device = torch.device("cuda:0")
    probe = ops.ClockProbe(device, capacity=4)
    x = torch.randn((4096, 4096), device=device)
    x = torch.tanh(x @ x * 1e-3)  # library load and first call outside the window
    torch.cuda.synchronize()
    a = probe.mark()
    for _ in range(40):
        x = torch.tanh(x @ x * 1e-3)
    b = probe.mark()
    torch.cuda.synchronize()
    ghz = probe.ghz(a, b)
    print("clock GHz per XCD", ghz, "counter spread", probe.spread(a), flush=True)
    assert len(ghz) >= 1
    # a busy window on MI355X runs between ~1 GHz and its 2.4 GHz peak
    assert all(0.5 < v < 3.0 for v in ghz.values()), ghz
    # readings of one CU's counter within one probe are microseconds apart
    assert probe.spread(a) < 100_000
    with pytest.raises(ValueError):
        for _ in range(5):
            probe.mark()
