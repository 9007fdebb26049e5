"""Lifetime rules for the HIP graphs that the serving engine and the graphed train step capture.

The HIP runtime does not allow a graph to be destroyed while another capture is in progress
on the process. A graph object is destroyed when its last Python reference goes. Refcounting
alone never does that inside a capture window, because no captured function drops a graph.
Python's cyclic garbage collector can, though. It runs whenever allocation counts cross its
thresholds, so it could fire in the middle of a capture and collect an unreachable engine
whose graphs were kept alive only by a reference cycle. :func:`capture_window` closes that
gap deterministically: it collects what is already unreachable, then keeps the cyclic
collector off until the capture ends. Owners of graphs also release them explicitly with
``close()`` (or a ``with`` block), so a graph's end does not depend on the collector at all.
"""

from __future__ import annotations

import contextlib
import gc


@contextlib.contextmanager
def capture_window():
    """Context for one ``torch.cuda.graph`` capture: no cyclic garbage collection inside it."""
    was_enabled = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()
