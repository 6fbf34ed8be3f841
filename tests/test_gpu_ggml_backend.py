"""The ggml backend end to end on the GPU: registry lookup by name, buffer
allocation, GGUF upload, graph_compute of MUL_MAT nodes (GEMV and GEMM sizes,
batched activations), MUL_MAT_ID on 3-D expert weights (routing views, broadcast and per-slot
activations), tensor_get round trips, partial weight writes (one spanning two experts), the
supports_op contract, a scheduler-style CPU-fallback split (MUL_MAT | host TANH | MUL_MAT), the
failure paths (an allocation the device cannot hold, a graph with an unclaimed node) followed by
working graphs, and the dynamic-loading entry points, all checked against the CPU oracle by the
native driver."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("moe_host", ["0", "1"])
def test_backend_driver_json(moe_host):
    """moe_host 0: MUL_MAT_ID routed on the device (the default); 1: the ids read back to the host."""
    exe = os.path.join(ROOT, "crispembed_amd", "bin", "test-backend-mi355")
    env = dict(os.environ, MQ_GGML_MOE_HOST=moe_host)
    r = subprocess.run([exe, "mi355", "--json"], capture_output=True, text=True, timeout=300, env=env)
    print(r.stderr[-2000:])
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["name"].startswith("MI355X")
    assert out["cases"] >= 24
    assert out["max_rel_err"] <= 1e-4
    assert out["dl_score"] > 0
    for k in ("roundtrip_ok", "partial_write_ok", "batched_ok", "supports_op_ok", "moe_ok", "sched_split_ok",
              "failures_ok", "computed", "correct"):
        assert out[k] is True, k
    assert r.returncode == 0
