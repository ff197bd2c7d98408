"""Emulated test runs shared by the test modules (test infrastructure only).

A test module registers its cases at import time; the first module fixture
that asks for a result builds the emulated library once and starts every
registered run that a selected test needs (tests/conftest.py reads their
`emu_jobs` markers) at the same time, each run one single-threaded child
process, so the CPU suite waits for the slowest run rather than the sum.
Collection alone starts nothing.
"""
from __future__ import annotations

import atexit
import json
from typing import Dict, List, Optional, Set, Tuple

from tests.emu import device

_REGISTERED: Dict[str, Tuple[List[str], float]] = {}
_STARTED: Dict[str, device.Child] = {}
_WANTED: Optional[Set[str]] = None     # jobs the selected tests need (None: all registered)


def want(names) -> None:
    """Restrict the runs started together to these (the selected tests' jobs)."""
    global _WANTED
    _WANTED = set(names)


@atexit.register
def _stop_unfinished() -> None:
    for c in _STARTED.values():
        if c.done is None and c.p.poll() is None:
            c.p.kill()


def register(name: str, cases: List[Tuple[str, dict]], timeout: float = 1800) -> None:
    args: List[str] = []
    for case, params in cases:
        args += [case, json.dumps(params)]
    _REGISTERED[name] = (args, timeout)


def result(name: str) -> Tuple[int, str, object]:
    if name not in _STARTED:
        for n, (args, timeout) in _REGISTERED.items():
            if n not in _STARTED and (n == name or _WANTED is None or n in _WANTED):
                _STARTED[n] = device.start_child("tests.emu.cases", args, timeout)
    return _STARTED[name].wait()
