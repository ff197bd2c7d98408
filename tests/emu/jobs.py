"""Emulated test runs shared by the test modules (test infrastructure only).

A test module registers its cases at import time; the first module fixture
that asks for a result builds the emulated library once and starts every
registered run at the same time (each run is one single-threaded child
process), so the CPU suite waits for the slowest run rather than the sum.
Collection alone starts nothing.
"""
from __future__ import annotations

import json
from typing import Dict, List, Tuple

from tests.emu import device

_REGISTERED: Dict[str, Tuple[List[str], float]] = {}
_STARTED: Dict[str, device.Child] = {}


def register(name: str, cases: List[Tuple[str, dict]], timeout: float = 1800) -> None:
    args: List[str] = []
    for case, params in cases:
        args += [case, json.dumps(params)]
    _REGISTERED[name] = (args, timeout)


def result(name: str) -> Tuple[int, str, object]:
    if name not in _STARTED:
        for n, (args, timeout) in _REGISTERED.items():
            if n not in _STARTED:
                _STARTED[n] = device.start_child("tests.emu.cases", args, timeout)
    return _STARTED[name].wait()
