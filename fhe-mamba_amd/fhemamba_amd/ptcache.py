"""Device-memory-bounded cache of encoded plaintexts.

Plaintexts of a CryptoContext of this package live in HBM (one limb of N
words per modulus of their level), so caches of encoded diagonals and masks
are bounded by bytes rather than by entries."""
from __future__ import annotations

from collections import OrderedDict


class PlaintextCache:
    """Encoded plaintexts (or lists of them) by key, least recently used
    first out once their device bytes pass the budget."""

    def __init__(self, ring_dim: int, budget: int):
        self.ring_dim, self.budget, self.bytes = int(ring_dim), int(budget), 0
        self._d: OrderedDict = OrderedDict()

    def _size(self, value) -> int:
        items = value if isinstance(value, list) else [value]
        total = 0
        for pt in items:
            poly = getattr(pt, "poly", None)
            total += 1 if poly is None else poly.npoly * poly.nlimb * self.ring_dim * 8
        return total

    def __len__(self) -> int:
        return len(self._d)

    def get(self, key):
        v = self._d.get(key)
        if v is not None:
            self._d.move_to_end(key)
            return v[0]
        return None

    def put(self, key, value) -> None:
        size = self._size(value)
        if key in self._d:
            self.bytes -= self._d.pop(key)[1]
        self._d[key] = (value, size)
        self.bytes += size
        while self.bytes > self.budget and len(self._d) > 1:
            _, (_, old) = self._d.popitem(last=False)
            self.bytes -= old
