"""Execution accounting of a runtime (eoship_accounting_read): the per-step
keys the reference's executor reports (device_execution, execution_mode,
uploaded_bytes, downloaded_bytes, sync_count; runtime/backend/symbolic.go:
174-216) counted exactly for a TurboQuant top-k on host arrays and on device
buffers."""
import numpy as np
import pytest

from eos_amd import datagen
from eos_amd.runtime import DeviceBuffer
from eos_amd.turboquant import TurboQuantIndex

pytestmark = pytest.mark.gpu


def test_accounting_counts_copies_syncs_and_launches(rt):
    print("[case] accounting of a TurboQuant top-k", flush=True)
    c = datagen.TurboQuantCorpus(20000, 384, 4, 3, 4, 5)
    q = datagen.baseline_queries(64, 384)
    idx = TurboQuantIndex(rt, c.codes, c.norms, c.dim, c.bits, c.codebook, c.codebook_scale,
                          c.rotation)
    rt.sync()
    base = rt.accounting(reset=True)
    assert base["device_execution"] and base["execution_mode"] == "hip_device"
    ids, sc, st = idx.top_k(q, 100)
    a = rt.accounting(reset=True)
    assert st.fallback_queries == 0
    assert a["uploaded_bytes"] == 64 * 384 * 4
    # per batch: status + kept counts (stats); then ids and scores
    assert a["downloaded_bytes"] == 64 * 4 + 64 * 4 + 64 * 100 * 8 + 64 * 100 * 4
    assert a["sync_count"] == 2
    assert a["kernel_launches"] >= 7
    assert a["graph_captures"] == 0 and a["graph_replays"] == 0
    # device buffers, no stats: nothing crosses PCIe and the host never waits
    dq = DeviceBuffer.from_array(rt, q)
    di, ds = DeviceBuffer(rt, 64 * 100 * 8), DeviceBuffer(rt, 64 * 100 * 4)
    rt.sync()
    rt.accounting(reset=True)
    idx.top_k_device(dq, 64, 100, di, ds, with_stats=False)
    b = rt.accounting(reset=True)
    assert (b["uploaded_bytes"], b["downloaded_bytes"], b["sync_count"]) == (0, 0, 0)
    assert b["kernel_launches"] == a["kernel_launches"] + 2  # gated fallback: dense + select
    for buf in (dq, di, ds):
        buf.free()
    idx.release()
