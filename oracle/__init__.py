"""CPU oracle (test infrastructure only; see reference_cpu.py's header)."""

from .reference_cpu import *  # noqa: F401,F403
