"""MI355X (gfx950) implementation of relmo's relational message-passing ops.

``relmo_amd.mp`` mirrors ``relmo.ops.mp`` for ``fanout_scatter``,
``fanin_reduce`` and the four pack ops that prepare their operands
(``fanout_pack_multi``, ``fanin_pack_multi``, ``fanout_pack_from_edges``,
``fanin_pack_from_edges``); the ops run on hand-written HIP kernels through
``relm_mp_ops.so`` (torch binding) and ``librelm_mp_hip.so`` (C ABI).
"""

from . import mp

__all__ = ["mp"]
