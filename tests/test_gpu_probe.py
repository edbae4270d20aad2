"""The issue-rate probe of the flash tile's instruction mix
(``fjx_probe_issue_mix``): every mix runs and reports a positive time, a
mix's time grows with its iteration count, and a superset mix is not faster
than its parts."""

from __future__ import annotations

import pytest

from foldjax_amd import _lib
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def test_issue_mix_probe_times():
    say("issue mix probe")
    t = {mix: _lib.probe_issue_mix(mix, 2, 400) for mix in range(5)}
    assert all(v > 0 for v in t.values()), t
    assert _lib.probe_issue_mix(2, 2, 1600) > 2.0 * t[2]
    assert t[0] >= 0.9 * max(t[2], t[3]), t  # the full mix contains the MFMAs and the exponentials
    with pytest.raises(ValueError):
        _lib.probe_issue_mix(5, 2, 10)
