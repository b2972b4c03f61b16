"""Host model of the decode step's exchange and last-arriver protocol (CPU only).

``tests/protocol_model.cpp`` runs the protocol of transformer_amd/csrc/msdecode.hip with
one std::thread per workgroup and std::atomic words: tagged exchange words polled until
their epoch tag matches, a 64-bit atomic max for the argmax, and a 32-bit arrival counter
whose last arrival publishes the token.  The kernel's rule (workgroup 0 resets the counter
and the key at the start of every step) must publish exactly one correct token per step
from any leftover state, across the 2**32 wrap of the counter and the epoch wrap; the
rule the kernel used before (never reset, publisher = arrival with old % GR == GR - 1)
is kept as a negative control and must fail once the counter nears 2**32 (with 240 row
workgroups, 2**32 is not a multiple of GR).
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("pm") / "protocol_model")
    subprocess.run([gxx, "-O2", "-std=c++17", "-pthread", "-o", exe, os.path.join(HERE, "protocol_model.cpp")],
                   check=True)
    return exe


def _run(exe, rule, gr, steps, counter, key, epoch, seed=1):
    r = subprocess.run([exe, rule, str(gr), str(steps), hex(counter), hex(key), hex(epoch), str(seed)],
                       capture_output=True, text=True, timeout=120)
    lines = r.stdout.strip().splitlines()
    steps_out = [dict(zip(ln.split()[0::2], ln.split()[1::2])) for ln in lines if ln.startswith("step")]
    return r.returncode, lines[-1], steps_out


@pytest.mark.parametrize("gr", [240, 252, 7])
def test_reset_rule_publishes_once_from_any_leftover_state(model, gr):
    # counter 16 below the 32-bit wrap, garbage argmax key, epochs crossing 0xFFFFFFFE -> 1
    rc, last, st = _run(model, "reset", gr, 5, 2**32 - 16, 0xDEADBEEFCAFEF00D, 0xFFFFFFFC)
    assert rc == 0 and last == "ok", st
    assert [s["epoch"] for s in st][2:4] == ["1", "2"]
    assert all(s["publishers"] == "1" and s["token"] == s["expected"] for s in st)


def test_modulo_rule_from_zeroed_workspace_works(model):
    rc, last, st = _run(model, "modulo", 240, 3, 0, 0, 5)
    assert rc == 0 and last == "ok", st


def test_modulo_rule_breaks_at_the_counter_wrap(model):
    """Negative control: 2**32 - 16 arrivals earlier (about 17.9M steps of 240 workgroups),
    the old rule publishes no token in one step and an early token in the next."""
    rc, last, st = _run(model, "modulo", 240, 3, 2**32 - 16, 0, 5)
    assert rc != 0 and last == "FAILED"
    assert st[0]["publishers"] == "0"
