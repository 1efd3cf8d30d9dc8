"""Graph capture and replay of the fused ops (slhip_graph_*): every replay equals the eager result, with
eager work and synchronizations between replays."""
import numpy as np
import pytest

import oracle
from sharplight_amd import native, synth
from tests.devutil import Dev, log
from tests.parity import assert_bf16_close, assert_bits_equal

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(device):
    c2 = synth.c2(rows=256)
    c3 = synth.c3(rows=64, cols=4096)
    c5 = synth.c5("q4_0", V=500, N=128)
    st = native.Stream()
    with Dev() as d:
        px, pr, pw = d.put(c2["x"]), d.put(c2["res"]), d.put(c2["w"])
        py, ph = d.empty(c2["x"].nbytes), d.empty(c2["x"].nbytes)
        pg, pu, po = d.put(c3["gate"]), d.put(c3["up"]), d.empty(c3["gate"].nbytes)
        pt, pi, pe = d.put(c5["table"]), d.put(c5["ids"]), d.empty(128 * 4096 * 2)

        def record():
            native.rownorm("rms", "bf16", "bf16", px, py, 256, 4096, res=pr, w=pw, h_out=ph, eps=c2["eps"],
                           stream=st.handle)
            native.gated_act("silu", "bf16", "bf16", pg, pu, po, 64, 4096, stream=st.handle)
            native.gather("q4_0", pt, 500, 4096, pi, 128, "bf16", pe, stream=st.handle)

        log("graph capture")
        g = native.Graph(st, record)
        yref, href = oracle.add_rmsnorm(c2["x"], c2["res"], c2["w"], c2["eps"], dtype="bf16")
        oref = oracle.gated("silu", c3["gate"], c3["up"], dtype="bf16")
        eref = oracle.gather_as("q4_0", c5["table"], 500, 4096, c5["ids"], dtype="bf16")
        for rep in range(4):
            for p, n in ((py, c2["x"].nbytes), (ph, c2["x"].nbytes), (po, c3["gate"].nbytes), (pe, 128 * 4096 * 2)):
                native.call("slhip_memset", p, 0x5A, n, st.handle)  # eager work between replays
            st.sync()
            log(f"graph replay {rep}")
            g.launch(st)
            st.sync()
            assert_bf16_close(d.get(py, (256, 4096), np.uint16), yref, what=f"replay {rep} y")
            assert_bf16_close(d.get(ph, (256, 4096), np.uint16), href, ulp=0, what=f"replay {rep} h")
            assert_bf16_close(d.get(po, (64, 4096), np.uint16), oref, what=f"replay {rep} swiglu")
            assert_bits_equal(d.get(pe, (128, 4096), np.uint16), eref, what=f"replay {rep} gather")
        del g


_FIRST_CALL_CAPTURED = r'''
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from sharplight_amd import native, synth
import oracle
# No slhip_set_device and no eager gather before the capture: the gather inside the graph is the first
# library call that needs the device's index-error word.
c = synth.c5("q8_0", V=300, N=64)
st = native.Stream()
pt, pi = native.DeviceBuffer.from_numpy(c["table"]), native.DeviceBuffer.from_numpy(c["ids"])
py = native.DeviceBuffer(64 * 4096 * 2)
native.synchronize()
g = native.Graph(st, lambda: native.gather("q8_0", pt, 300, 4096, pi, 64, "bf16", py, stream=st.handle))
for _ in range(3):
    g.launch(st)
    st.sync()
    got = py.download((64, 4096), np.uint16)
    ref = oracle.gather_as("q8_0", c["table"], 300, 4096, c["ids"], dtype="bf16")
    assert np.array_equal(got, ref)
bad = c["ids"].copy()
bad[5] = 300
pi.upload(bad)
native.synchronize()
g.launch(st)
try:
    st.sync()
    raise SystemExit("no index error")
except IndexError as e:
    assert "300" in str(e), e
print("ok")
'''


def test_first_gather_under_capture_needs_no_allocation(device, tmp_path):
    """The gather index-error word is a device variable: a gather captured before any other library call
    on the device (so nothing could have allocated for it) records, replays and reports a bad id."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "first_call.py"
    script.write_text(_FIRST_CALL_CAPTURED)
    log("subprocess: first gather under capture")
    r = subprocess.run([sys.executable, str(script), root], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
