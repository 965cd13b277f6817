"""CPU oracle of the prefix cache -- TEST INFRASTRUCTURE ONLY.

A plain-Python restatement of the reference's ``PagedPrefixCache``
(``include/helix/kv_cache/prefix.hpp:66-112``, ``src/kv_cache/prefix.cpp``)
over any pool object with ``fork_sequence(seq, tokens)``,
``release_sequence(seq)``, ``length(seq)`` and ``block_tokens``.  The
reference's digest index only speeds candidate search; every match is
verified against the exact token vector (prefix.cpp:143-149, 380-387), so
the observable behaviour is exact-key matching, which is what this states
directly: a most-recently-used list of entries scanned linearly.  Only
``tests/`` imports it.
"""

from __future__ import annotations

from . import INVALID_ARGUMENT, OUT_OF_RANGE, OracleError

INSERTED, ALREADY_PRESENT, REJECTED_TOO_LARGE = 0, 1, 2
_U64_MAX = (1 << 64) - 1

STAT_NAMES = (
    "maximum_entries", "maximum_block_references", "entry_count", "retained_tokens",
    "retained_block_references", "peak_entries", "peak_block_references",
    "lookup_count", "hit_count", "miss_count", "insertion_count", "duplicate_insertion_count",
    "rejected_insertion_count", "eviction_count", "erase_count")


class PrefixCacheOracle:
    def __init__(self, pool, maximum_entries, maximum_block_references):
        # prefix.cpp:124-139.
        if pool is None:
            raise OracleError(INVALID_ARGUMENT, "paged cache must not be null")
        if maximum_entries == 0 or maximum_block_references == 0:
            raise OracleError(INVALID_ARGUMENT, "limits must be positive")
        self.pool = pool
        self.page = pool.block_tokens
        if maximum_block_references > _U64_MAX // self.page:
            raise OracleError(OUT_OF_RANGE, "retained token accounting would overflow")
        self.max_entries = maximum_entries
        self.max_blocks = maximum_block_references
        self.entries = []  # most recent first: [namespace, tokens tuple, anchor, blocks]
        self.s = {n: 0 for n in STAT_NAMES}
        self.s["maximum_entries"] = maximum_entries
        self.s["maximum_block_references"] = maximum_block_references

    def _bump(self, name):
        if self.s[name] != _U64_MAX:
            self.s[name] += 1

    def _validate(self, ns, tokens):
        # prefix.cpp:151-161.
        if ns == 0 or len(tokens) == 0 or len(tokens) % self.page != 0:
            raise OracleError(INVALID_ARGUMENT, "invalid prefix key")

    def _find(self, ns, tokens):
        key = tuple(tokens)
        for i, e in enumerate(self.entries):
            if e[0] == ns and e[1] == key:
                return i
        return -1

    def _erase_at(self, i, eviction):
        # prefix.cpp:164-186.
        ns, key, anchor, blocks = self.entries[i]
        self.pool.release_sequence(anchor)
        del self.entries[i]
        self.s["retained_tokens"] -= len(key)
        self.s["retained_block_references"] -= blocks
        self.s["entry_count"] -= 1
        self._bump("eviction_count" if eviction else "erase_count")

    def insert(self, ns, tokens, source, source_length):
        """``source_length`` is the pool's length of ``source`` (the caller
        raises for a foreign or released source, as ``cache->length`` does)."""
        # prefix.cpp:296-358.
        self._validate(ns, tokens)
        if len(tokens) > source_length:
            raise OracleError(OUT_OF_RANGE, "prefix exceeds the source sequence length")
        i = self._find(ns, tokens)
        if i >= 0:
            self.entries.insert(0, self.entries.pop(i))
            self._bump("duplicate_insertion_count")
            return ALREADY_PRESENT
        blocks = len(tokens) // self.page
        if blocks > self.max_blocks:
            self._bump("rejected_insertion_count")
            return REJECTED_TOO_LARGE
        anchor = self.pool.fork_sequence(source, len(tokens))
        self.entries.insert(0, [ns, tuple(tokens), anchor, blocks])
        # prefix.cpp:188-198: the list size counts the new entry, the retained
        # statistic does not yet.
        while (len(self.entries) > self.max_entries
               or self.s["retained_block_references"] > self.max_blocks - blocks):
            assert len(self.entries) > 1
            self._erase_at(len(self.entries) - 1, True)
        self.s["entry_count"] += 1
        self.s["retained_tokens"] += len(tokens)
        self.s["retained_block_references"] += blocks
        self.s["peak_entries"] = max(self.s["peak_entries"], self.s["entry_count"])
        self.s["peak_block_references"] = max(self.s["peak_block_references"],
                                              self.s["retained_block_references"])
        self._bump("insertion_count")
        return INSERTED

    def lookup_longest(self, ns, tokens, maximum_prefix_tokens=None):
        # prefix.cpp:360-403.
        if ns == 0:
            raise OracleError(INVALID_ARGUMENT, "prefix namespace zero is reserved as invalid")
        bound = len(tokens) if maximum_prefix_tokens is None else min(len(tokens),
                                                                      maximum_prefix_tokens)
        aligned = bound - bound % self.page
        best, best_tokens = -1, 0
        for n in range(self.page, aligned + 1, self.page):
            i = self._find(ns, tokens[:n])
            if i >= 0:
                best, best_tokens = i, n
        if best < 0:
            self._bump("lookup_count")
            self._bump("miss_count")
            return None
        entry = self.entries[best]
        seq = self.pool.fork_sequence(entry[2], best_tokens)
        self.entries.insert(0, self.entries.pop(best))
        self._bump("lookup_count")
        self._bump("hit_count")
        return seq, best_tokens

    def contains(self, ns, tokens):
        self._validate(ns, tokens)
        return self._find(ns, tokens) >= 0

    def erase(self, ns, tokens):
        self._validate(ns, tokens)
        i = self._find(ns, tokens)
        if i < 0:
            return False
        self._erase_at(i, False)
        return True

    def evict_lru(self):
        if not self.entries:
            return False
        self._erase_at(len(self.entries) - 1, True)
        return True

    def clear(self):
        while self.entries:
            self._erase_at(len(self.entries) - 1, False)

    def stats(self):
        return dict(self.s)
