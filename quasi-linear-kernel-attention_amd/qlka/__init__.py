"""Shared native layer of the MI355X weighted_abs_sum / weighted_laplace_sum operators (libqlka.so).

`qlka.ops` exposes the test entry points of the C ABI (segmented sort, merge rank); the operator entry points live in
the drop-in packages `weighted_abs_sum` and `weighted_laplace_sum` next to this one.
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
