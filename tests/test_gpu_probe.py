"""The measurement probes. The issue-rate probe of the flash tile's
instruction mix (``fjx_probe_issue_mix``): every mix runs and reports a
positive time, a mix's time grows with its iteration count, and a superset
mix is not faster than its parts. The HBM streaming probe
(``fjx_probe_hbm_stream``): every mode runs at a plausible rate."""

from __future__ import annotations

import pytest

from foldjax_amd import _lib
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def test_issue_mix_probe_times():
    say("issue mix probe")
    t = {mix: _lib.probe_issue_mix(mix, 2, 400) for mix in range(7)}
    assert all(v > 0 for v in t.values()), t
    assert _lib.probe_issue_mix(2, 2, 1600) > 2.0 * t[2]
    assert t[0] >= 0.9 * max(t[2], t[3]), t  # the full mix contains the MFMAs and the exponentials
    assert t[5] >= 0.9 * max(t[6], t[3]), t  # so does its 32x32x16 form
    with pytest.raises(ValueError):
        _lib.probe_issue_mix(7, 2, 10)


def test_hbm_stream_probe_rates():
    """``fjx_probe_hbm_stream``: every mode runs, a copy moves twice the bytes
    of a read in more time than the read, and the rates sit below the 8 TB/s
    figure (a probe that reported more would be timing nothing)."""
    say("hbm stream probe")
    nbytes = 256 << 20
    t = {mode: _lib.probe_hbm_stream(mode, 2, nbytes) for mode in range(4)}
    assert all(v > 0 for v in t.values()), t
    assert t[0] > t[2], t
    for mode, ms in t.items():
        moved = nbytes * (2 if mode in (0, 1) else 1)
        assert moved / (ms * 1e-3) < 8.0e12, (mode, ms)
    with pytest.raises(ValueError):
        _lib.probe_hbm_stream(4, 2, nbytes)
    with pytest.raises(ValueError):
        _lib.probe_hbm_stream(0, 2, 1000)
