"""MI355X (gfx950) implementation of GMDN's chunkwise fast-weight state scan.

* ``gmdn_amd.scan``   -- the drop-in chunk state scan op (``fast_state_scan``)
* ``gmdn_amd.chunk``  -- the fused mixer-core op (q, k, v, beta, log-gates -> o)
* ``gmdn_amd.build``  -- hipcc recipe of the C-ABI library ``libgmdn_scan.so``

The reference-compatible module is ``fast_scan`` one directory up.
"""
from . import _native  # noqa: F401

__all__ = ["_native"]
