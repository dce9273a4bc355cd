"""A process that ends with a context still open exits cleanly. An engine that failed between ss_open and ss_close
(an exception after the open) leaves a device-gated context with a live service thread, its streams and its mapped
words; the library closes every context still open from an exit handler registered at the first ss_open, which runs
before the HIP runtime's own finalizers. Each case runs in a child process and must end with the child's own exit
status (1: the uncaught exception), never a signal. dg-mid-token: the engine fails after ss_begin with a token's
export and wait kernels enqueued and no ss_end (a low dg_wait_timeout_ms): closing stops the service and raises the
host abort, on which every wait kernel of the token ends."""
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = textwrap.dedent("""
    import sys
    sys.path.insert(0, {root!r})
    import numpy as np
    import tierstream_amd as tsa
    from oracle import fixtures
    from tierstream_amd import ss

    tsa.check(tsa.lib().tsa_set_device(0))
    KiB = 1024
    mode = {mode!r}
    m = fixtures.write_model({tmp!r}, 3, 8, [64 * KiB] * 3, top_k=2, seed=5)
    st = (m.unit_bytes + 255) // 256 * 256
    hs = (m.unit_bytes + 4095) // 4096 * 4096
    d = ss.Desc(m.desc_json())
    if mode in ("dg", "dg-mid-token"):
        bkw = dict(device_bytes=(12 + 5 + 3) * st + st // 2, host_pinned_bytes=(24 - 12 + 6 + 5) * hs + (64 << 20),
                   dynamic_slots_per_layer=1, ring_slots=5, tier_mode=1, host_spare_units=6)
        ctx = ss.Ctx(d, ss.budget(**bkw), ss.Plan(d, ss.budget(**bkw)),
                     ss.options(forward_mode=1, dg_max_ids=2, pin_planned=0, verify_hash=2,
                                dg_wait_timeout_ms=1000 if mode == "dg-mid-token" else 5000))
        eng = ss.DgEngine(ctx, 2, use_graph=True)
        rng = np.random.default_rng(3)
        for t in range(3):
            eng.token(np.stack([rng.choice(8, size=2, replace=False) for _ in range(3)]).astype(np.int32))
        if mode == "dg-mid-token":
            eng.token_open(np.stack([rng.choice(8, size=2, replace=False) for _ in range(3)]).astype(np.int32))
            print("token open", flush=True)
    else:
        bkw = dict(device_bytes=10 * st + 8 * st + st // 2, host_pinned_bytes=24 * hs + (8 << 20), ring_slots=8)
        ctx = ss.Ctx(d, ss.budget(**bkw), None, ss.options())
        ctx.host_run(fixtures.uniform_routes(3, 8, 2, 3, seed=4), 0)
    print("tokens done; leaving the context open", flush=True)
    raise RuntimeError("engine failure after ss_open")
""")


@pytest.mark.parametrize("mode", ["dg", "dg-mid-token", "host"])
def test_exit_with_an_open_context(tmp_path, gpu, mode):
    script = tmp_path / "child.py"
    script.write_text(CHILD.format(root=str(ROOT), tmp=str(tmp_path), mode=mode))
    p = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=180,
                       env={**os.environ, "PYTHONUNBUFFERED": "1"})
    assert "tokens done" in p.stdout, (p.returncode, p.stdout, p.stderr[-2000:])
    assert mode != "dg-mid-token" or "token open" in p.stdout, p.stdout
    assert p.returncode == 1, (p.returncode, p.stderr[-2000:])  # the exception's status, not a signal
    assert "RuntimeError: engine failure after ss_open" in p.stderr, p.stderr[-2000:]
