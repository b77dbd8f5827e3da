"""Context workspaces: rf_ctx_reserve sizes them up front; with a fixed
reservation no call allocates (a call that needs more is refused), growth is
refused during graph capture, and a graph captured before a workspace was
replaced is refused at replay instead of reading the freed buffer."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _attention_inputs(c, rng, hist, qh=32, kvh=8, hd=128):
    arrs = [rng.normal(0, 1, n).astype(np.float32)
            for n in (qh * hd, max(hist, 1) * kvh * hd, max(hist, 1) * kvh * hd, kvh * hd, kvh * hd)]
    return [c.array(a) for a in arrs]


def test_fixed_reservation_allocates_nothing():
    import ramforge_amd as rf

    rng = np.random.default_rng(31)
    with rf.Context(0) as c:
        # up to 64 positions: 8 chunks per query head at most (the split
        # records of 32 heads, hd + 4 floats each), more than the any-shape
        # kernel's score rows
        need = c.attention_workspace_bytes(64, 32, 8, 128)
        assert need == 8 * 32 * 132 * 4
        dev = _attention_inputs(c, rng, 8191)
        out = c.empty((32 * 128,))
        c.reserve(attention_bytes=need, fixed=True)
        used = c.vram_used
        for hist in (63, 40, 0):
            print(f"  reserved attention hist={hist}", flush=True)
            rf.attention_checked(c, *dev, hist, 32, 8, 128, out=out)
            c.synchronize()
            assert c.vram_used == used, hist
        # 2048 positions take 32 chunks per KV head: more than reserved
        with pytest.raises(rf.RamforgeError, match="fixed"):
            rf.attention_checked(c, *dev, 2047, 32, 8, 128, out=out)
        assert c.vram_used == used
        # a larger reservation lifts the limit again
        c.reserve(attention_bytes=c.attention_workspace_bytes(8192, 32, 8, 128), fixed=True)
        rf.attention_checked(c, *dev, 8191, 32, 8, 128, out=out)
        c.synchronize()


def test_matmul_reservation_covers_the_call():
    import ramforge_amd as rf
    from helpers import Q8_0, pack_host, random_matrix

    rng = np.random.default_rng(32)
    rows, k, n = 512, 1024, 80  # two launches: 64 tokens and a remainder of 16
    raw = random_matrix(Q8_0, rows, k, rng)
    with rf.Context(0) as c:
        w = c.array(pack_host(Q8_0, raw, rows, k))
        x = c.array(rng.normal(0, 1, (n, k)).astype(np.float32))
        y = c.empty((n, rows))
        c.reserve(matmul_bytes=c.matmul_workspace_bytes(rows, k, n), fixed=True)
        used = c.vram_used
        rf.matmul_packed(c, Q8_0, w, (rows, k), x, n, y)
        c.synchronize()
        assert c.vram_used == used


def test_growth_refused_during_capture():
    import ramforge_amd as rf

    rng = np.random.default_rng(33)
    with rf.Context(0) as c:
        dev = _attention_inputs(c, rng, 4095)
        out = c.empty((32 * 128,))
        with pytest.raises(rf.RamforgeError, match="during graph capture"):
            with c.capture():
                rf.attention_checked(c, *dev, 4095, 32, 8, 128, out=out)
        # outside a capture the same call grows the workspace and runs
        rf.attention_checked(c, *dev, 4095, 32, 8, 128, out=out)
        c.synchronize()


def test_stale_graph_refused_after_workspace_growth():
    import ramforge_amd as rf

    rng = np.random.default_rng(34)
    with rf.Context(0) as c:
        dev = _attention_inputs(c, rng, 8191)
        out = c.empty((32 * 128,))
        rf.attention_checked(c, *dev, 100, 32, 8, 128, out=out)  # sizes the workspace
        c.synchronize()
        with c.capture() as cap:
            rf.attention_checked(c, *dev, 100, 32, 8, 128, out=out)
        g = cap.graph
        g.replay(2)
        want = out.numpy()
        rf.attention_checked(c, *dev, 8191, 32, 8, 128, out=out)  # replaces the workspace
        c.synchronize()
        with pytest.raises(rf.RamforgeError, match="captured before"):
            g.replay(1)
        g.close()
        with c.capture() as cap2:  # a new capture uses the new buffer
            rf.attention_checked(c, *dev, 100, 32, 8, 128, out=out)
        cap2.graph.replay(2)
        assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32))
        cap2.graph.close()


_SETUP_SCRIPT = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import ramforge_amd as rf
from ramforge_amd import GGML

rng = np.random.default_rng(35)
rows, k = 96, 4096
raw = rng.integers(0, 256, size=(rows, k // 32, 34), dtype=np.uint8)
raw[:, :, 0:2] = np.frombuffer(np.full(rows * k // 32, 0x2000, np.uint16).tobytes(), np.uint8).reshape(rows, -1, 2)
with rf.Context(0) as c:
    w = c.array(raw.reshape(-1))
    p = c.empty((raw.size,), "uint8")
    rf.pack_weights(c, GGML.Q8_0, w, rows, k, p)
    x = c.array(rng.normal(0, 1, k).astype(np.float32))
    y = c.empty((rows,))
    # the first launch of this kernel shape in the process: its setup
    # (dynamic LDS attribute, occupancy) is refused inside a capture
    try:
        with c.capture():
            rf.matvec_packed(c, GGML.Q8_0, p, (rows, k), x, y)
        print("captured without refusal")
        sys.exit(1)
    except rf.RamforgeError as e:
        assert "inside a stream capture" in str(e), str(e)
    # once launched outside a capture, the same shape captures and replays
    rf.matvec_packed(c, GGML.Q8_0, p, (rows, k), x, y)
    c.synchronize()
    want = y.numpy()
    y.upload(np.zeros(rows, np.float32))
    with c.capture() as cap:
        rf.matvec_packed(c, GGML.Q8_0, p, (rows, k), x, y)
    cap.graph.replay(2)
    assert np.array_equal(y.numpy().view(np.uint32), want.view(np.uint32))
    cap.graph.close()
print("ok")
"""


def test_first_launch_setup_refused_inside_capture():
    """A launcher's one-time kernel setup (dynamic LDS attribute, occupancy
    query) is never made inside a stream capture: the first launch of a
    kernel shape inside a capture is refused with a clear error, and the
    same shape captures and replays once it has run outside.  Run in a fresh
    process, where no shape has been set up yet."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _SETUP_SCRIPT, root], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
