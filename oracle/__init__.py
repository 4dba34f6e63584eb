"""CPU oracle package — test infrastructure only (see oracle/oracle.py's header)."""
from .oracle import *  # noqa: F401,F403
from .oracle import build, lib  # noqa: F401
