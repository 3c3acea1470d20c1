"""The C++ engine API on the GPU: tests/cpp/engine_greedy, a host program
built on include/neon_engine.hpp (neon::Engine over libneon_gptoss.so),
runs init_random -> prefill -> decode and checks every greedy id and the
last step's fp32 logits against the CPU oracle it links as the checker.  The
program is built by __graft_entry__.build() (make -C tests/cpp)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "engine_greedy")


@pytest.mark.parametrize("shape,steps,batch", [("small", 32, 2), ("20b", 8, 1)])
def test_cpp_engine_greedy_matches_oracle(shape, steps, batch):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (run __graft_entry__.build())")
    print(f"engine_greedy {shape} steps={steps} batch={batch}", flush=True)
    r = subprocess.run([EXE, shape, str(steps), str(batch)], capture_output=True, text=True,
                       timeout=300)
    sys.stdout.write(r.stdout + r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 id mismatches; last logits bit-identical" in r.stdout
