"""Plants mistakes in the oracle (on the CPU) and checks that the pins catch
each one. oracle.c has -DORC_MUTANT=<k> hooks; each mutant is built with the
same flags as the real oracle into a temporary directory.

 1  log-sum-exp without the running max        5  dK accumulates k_j instead of q_i
 2  Delta term dropped from dS                 6  dQ missing the softmax scale
 3  Delta term with the wrong sign
 4  dV indexed by the key row of dO (transposed index)
"""
from __future__ import annotations

import os
import subprocess

import pytest

import oracle
from oracle_pins import all_pins

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle",
                   "oracle.c")


def _build(tmp_path, mutant):
    out = os.path.join(str(tmp_path), f"liboracle_m{mutant}.so")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-std=c11",
                    "-shared", f"-DORC_MUTANT={mutant}", "-o", out, SRC, "-lm", "-lpthread"],
                   check=True)
    return oracle.load(out)


def test_unmutated_build_passes_every_pin(tmp_path):
    lib = _build(tmp_path, 0)
    assert lib.orc_mutant() == 0
    assert all_pins(lib) == {}


@pytest.mark.parametrize("mutant", [1, 2, 3, 4, 5, 6])
def test_mutant_fails_a_pin(tmp_path, mutant):
    lib = _build(tmp_path, mutant)
    assert lib.orc_mutant() == mutant
    failed = all_pins(lib)
    assert failed, f"mutant {mutant} passed every pin"
