"""The host-thread model of the ring-queue protocol (tests/queue_model/queue_model.cpp).

The model restates the protocol of gpu-pipes_amd/csrc/pipes.hpp with
std::thread workgroups and std::atomic counters: epoch-tagged full / empty
counters, the epoch lift on a slot's first round, the NP / NC wait targets,
split round robin, row counts, and bounded waits with an epoch-tagged error
word.  It must pass its scenarios (1:1, broadcast, split / merge, four
column producers, two row-half producers of a one-slot queue, partial tiles, back-to-back launches over garbage from
older launches, a stuck producer) both as a plain build and under
ThreadSanitizer, and each planted protocol mistake must be caught.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "queue_model", "queue_model.cpp")


def build(tmp_path, tsan):
    exe = str(tmp_path / ("qm_tsan" if tsan else "qm"))
    cmd = ["g++", "-std=c++17", "-pthread", SRC, "-o", exe]
    cmd[1:1] = ["-O1", "-g", "-fsanitize=thread"] if tsan else ["-O2"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


@pytest.fixture(scope="module")
def exes(tmp_path_factory):
    d = tmp_path_factory.mktemp("queue_model")
    return {"plain": build(d, False), "tsan": build(d, True)}


def run(exe, mutant=0):
    return subprocess.run([exe, str(mutant)], capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("kind", ["plain", "tsan"])
def test_protocol_scenarios_pass(exes, kind):
    r = run(exes[kind])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all scenarios passed" in r.stdout
    assert "ThreadSanitizer" not in r.stderr


@pytest.mark.parametrize("mutant,what", [(1, "no epoch lift"), (2, "producer waits one round short"),
                                         (4, "split worker with the wrong stride"),
                                         (5, "consumer commits before reading"),
                                         (6, "row-half producers commit their own rows")])
def test_planted_protocol_mistakes_are_caught(exes, mutant, what):
    r = run(exes["plain"], mutant)
    assert r.returncode != 0, f"{what} went undetected: {r.stdout}"
    assert "FAILED" in r.stderr


def test_missing_release_is_a_data_race(exes):
    """Commits without release ordering: only ThreadSanitizer can see it."""
    r = run(exes["tsan"], 3)
    assert r.returncode != 0
    assert "ThreadSanitizer: data race" in r.stderr
