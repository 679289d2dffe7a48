"""Error paths on the GPU: a failing HIP call surfaces as EJ_E_HIP with a
message, raised by the Python wrappers, and leaves the library usable.  The
failure is injected from the host (EJ_INJECT_FAULT=launch makes every launch
check report hipErrorLaunchFailure while the kernel itself runs on valid
buffers), so no kernel faults."""

import numpy as np
import numpy.testing as npt
import pytest
import torch

from oracle import reference_path as R

import einjax_amd as ej

pytestmark = pytest.mark.gpu


def test_injected_launch_failure_then_recovery(gpu, monkeypatch):
    print("[case] EJ_INJECT_FAULT=launch on a valid segment_sum", flush=True)
    rng = np.random.default_rng(0)
    v = rng.standard_normal((40, 4, 4)).astype(np.float32)
    oc = rng.integers(0, 5, (40, 2)).astype(np.int32)
    dv, doc = torch.from_numpy(v).cuda(), torch.from_numpy(oc).cuda()
    monkeypatch.setenv("EJ_INJECT_FAULT", "launch")
    with pytest.raises(RuntimeError, match="HIP error in .*kernel launch failed.*injected"):
        ej.segment_sum(dv, doc)
    monkeypatch.delenv("EJ_INJECT_FAULT")
    torch.cuda.synchronize()
    coords, agg = ej.segment_sum(dv, doc)
    want_c, want_v = R.segment_sum(v, oc)
    npt.assert_array_equal(coords.cpu().numpy(), want_c)
    npt.assert_array_equal(agg.cpu().numpy(), want_v)
