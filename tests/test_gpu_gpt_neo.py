"""The engine's GPT-Neo with its attention answered by the device path.

oracle/_ref/engine_gpt_neo (built by `make -C oracle gpt_neo` from the engine's
headers and this repository's library) runs GPTNeo / Block::forward from the
engine, with Attention::context of the device model going through the C ABI:
the int8 prefill kernel for a prompt, the prefill over the device cache for a
later chunk of a prompt, the KV append and the decode kernel for one token. It
checks every attention call against the engine's own int8 attention composition on
the same inputs (max |diff| <= 1e-3), and, over whole models, prefill == decode for
40 prompt lengths and chunked prompts (six chunk schedules) == one token at a time
(max |dlogit| <= 1e-3), and the device
model against the engine's float model under 5% of the largest logit (the
engine's own bound for its W8A8 model, test_gpt_neo.cpp:167-187); it exits 0
when all hold. Skipped
where the program was not built (it needs the reference checkout at build
time)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "engine_gpt_neo")

pytestmark = pytest.mark.gpu


def test_engine_gpt_neo_with_device_attention():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not os.path.exists(BIN):
        pytest.skip("oracle/_ref/engine_gpt_neo not built (make -C oracle gpt_neo)")
    print("\n[case] engine GPT-Neo, attention through the device path", flush=True)
    proc = subprocess.run([BIN], capture_output=True, text=True, timeout=600)
    sys.stdout.write(proc.stdout)
    sys.stdout.write(proc.stderr)
    lines = [l for l in proc.stdout.splitlines() if l.startswith("{")]
    assert lines, "no summary line"
    rec = json.loads(lines[-1])
    assert rec["prefill_calls"] > 0 and rec["decode_calls"] > 0 and rec["chunk_calls"] > 0
    assert rec["call_max_diff"] <= 1e-3
    assert rec["prefill_decode_max_diff"] <= 1e-3
    assert rec["chunked_max_diff"] <= 1e-3
    assert rec["engine_max_diff"] <= 0.05 * rec["max_logit"]
    assert proc.returncode == 0
