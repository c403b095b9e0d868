"""Score-driven staging: keeps the engine's staging slots holding the
host-resident adapters a scheduler expects to need next.

The reference publishes per-adapter scheduler scores (Whittle index, GWAR
prediction, arrival rate) to the GPU every tick through its scheduler bridge
(csrc/bridge/warp_pipe_metadata.h:89-104, lora_warp_pipe/scheduler_bridge.py:
105-184), but no kernel or host path consumes them (csrc/kernels/
prefetch_kernel.cu:17-22): staging is driven by explicit prefetch_adapter
calls.  This policy is that consumer on the host side, over
the engine's own staging API (prefetch_adapter / is_prefetch_ready /
release_prefetch): each update ranks the candidates (the ids the next step
must have first, then by score, highest first, ties by id), keeps the top
`slots` staged, releases the rest, and issues prefetches for the newly
ranked ones on the engine's prefetch stream.  Scores are plain numbers per
adapter id; the bridge's own format is not part of this build.

The policy owns the slots it fills: prefetch or release the same adapters
elsewhere and its bookkeeping no longer matches the engine's.
"""
from typing import Dict, Hashable, Iterable, List, Optional


class ScorePrefetchPolicy:
    def __init__(self, engine, slots: Optional[int] = None, layer=None):
        """engine: a WarpPipeEngine whose candidates are host-resident
        (registered from CPU tensors).  slots: how many to keep staged
        (default: every staging slot of the engine).  layer: the adapters'
        layer in a multi-layer store (WarpPipeConfig.layer_stride)."""
        self.engine = engine
        self.slots = int(engine.config.num_staging_slots if slots is None else slots)
        if self.slots < 0:
            raise ValueError("slots must be >= 0")
        self.layer = layer
        self._staged: Dict[Hashable, int] = {}  # adapter id -> staging slot

    @property
    def staged(self) -> Dict[Hashable, int]:
        """Adapter id -> staging slot of what the policy keeps staged."""
        return dict(self._staged)

    def ranking(self, scores: Dict[int, float], must: Iterable[int] = ()) -> List[int]:
        """Candidates in staging order: `must` first (in the given order), then
        by score (highest first; ties by the smaller id)."""
        order = list(dict.fromkeys(int(a) for a in must))
        rest = sorted((int(a) for a in scores if int(a) not in set(order)), key=lambda a: (-float(scores[a]), a))
        return order + rest

    def update(self, scores: Dict[int, float], must: Iterable[int] = ()) -> List[int]:
        """Restages for the next step; returns the ids whose prefetch this
        call issued (the ones still staged from earlier calls are kept as
        they are).  An id the engine does not know, or one for which no slot
        is free, is skipped."""
        want = self.ranking(scores, must)[: self.slots]
        keep = set(want)
        for aid in [a for a in self._staged if a not in keep]:
            self.engine.release_prefetch(aid, layer=self.layer)
            del self._staged[aid]
        issued = []
        for aid in want:
            if aid in self._staged:
                continue
            slot = self.engine.prefetch_adapter(aid, layer=self.layer)
            if slot >= 0:
                self._staged[aid] = slot
                issued.append(aid)
        return issued

    def ready(self, adapter_id: int) -> bool:
        """True once the adapter's staged copy has landed."""
        return adapter_id in self._staged and self.engine.is_prefetch_ready(adapter_id, layer=self.layer)

    def release_all(self) -> None:
        for aid in list(self._staged):
            self.engine.release_prefetch(aid, layer=self.layer)
        self._staged.clear()
