"""The drop-in inside the engine's own code: oracle/_ref/engine_dropin runs the
Reef engine's operators (compiled from its headers) beside the device path called
through include/reef_hip/attention.hpp on the same inputs: Attention::context
(global and windowed), prompt append + decode == the last context row, the
integer-only head and the W8A8 projection bit-identical. The binary is built where
the engine headers are (make -C oracle dropin); elsewhere the test is skipped."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "oracle", "_ref", "engine_dropin")


def test_engine_dropin():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/engine_dropin was not built (needs the engine headers)")
    print("\n[case] engine drop-in program", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
