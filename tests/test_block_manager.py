"""Property tests of the KV block manager and prefix cache (host only).

The reference fixes the invariant these check (CLAUDE.md:71): every block is
either free or referenced by >= 1 block table, its refcount equals the
number of references, and nothing is freed while a running sequence uses it
("checked by property tests").  A hypothesis state machine drives random
admissions (prompts from a 3-letter alphabet, so prefixes collide often),
appends, forks and frees against a Python model of every live sequence's
tokens and of every block's contents, and after each step checks:
  * the manager's own exhaustive invariant check (refcounts, one state per
    block, cache index consistent);
  * each table covers its tokens: ceil(tokens / block_size) blocks;
  * an append's slot is slot_of(table, position) (paged.rs:47-52);
  * a prefix-cache hit only ever hands out a block whose whole prefix (its
    tokens and every token before it, which its KV at layers >= 1 depends
    on) equals the prompt's, also when block hashes are made to collide on
    purpose (the vo_bm_test_unchained_hash hook: a block hashes its own tokens
    only);
  * copy on write only copies a block another live sequence still uses, into
    a block nobody else uses;
  * blocks no live table references are all available again;
  * a request the pool cannot serve raises CapacityError and changes nothing.
"""
import numpy as np
import pytest
from hypothesis import HealthCheck, settings
from hypothesis import strategies as st
from hypothesis.stateful import RuleBasedStateMachine, initialize, invariant, precondition, rule

import __graft_entry__ as g

vo = g._load_package()


class BlockManagerMachine(RuleBasedStateMachine):
    unchained = False  # block hashes ignore the prefix (collisions on purpose)

    @initialize(num_blocks=st.integers(4, 40), bs=st.sampled_from([1, 2, 4, 16]),
                caching=st.booleans())
    def setup(self, num_blocks, bs, caching):
        self.bm = vo.BlockManager(num_blocks, bs, prefix_caching=caching)
        if self.unchained:
            self.bm.test_unchained_hash(True)
        self.N, self.bs, self.caching = num_blocks, bs, caching
        self.seqs = {}        # seq id -> list of tokens
        # block id -> the tokens up to the end of that full block (model): its
        # KV depends on all of them
        self.content = {}
        self.next_id = 0

    # -- helpers ----------------------------------------------------------
    def _table(self, s):
        return [int(b) for b in self.bm.block_table(s)]

    def _live_blocks(self):
        used = set()
        for s in self.seqs:
            used.update(self._table(s))
        return used

    def _record_full_blocks(self, s):
        toks, table = self.seqs[s], self._table(s)
        for i in range(len(toks) // self.bs):
            self.content[table[i]] = tuple(toks[:(i + 1) * self.bs])

    def _snapshot(self):
        return {s: self._table(s) for s in self.seqs}, self.bm.available()

    # -- rules ------------------------------------------------------------
    @rule(data=st.data())
    def add(self, data):
        n = data.draw(st.integers(1, 5 * self.bs))
        base = data.draw(st.sampled_from(list(self.seqs) + [None]))
        if base is not None and data.draw(st.booleans()):
            # share a prefix with a live sequence
            k = data.draw(st.integers(0, len(self.seqs[base])))
            toks = list(self.seqs[base][:k]) + data.draw(st.lists(st.integers(0, 2), min_size=0,
                                                                   max_size=n))
            if not toks:
                toks = [0]
        else:
            toks = data.draw(st.lists(st.integers(0, 2), min_size=1, max_size=n))
        need = -(-len(toks) // self.bs)
        sid = self.next_id
        self.next_id += 1
        before = self._snapshot()
        try:
            cached = self.bm.add_sequence(sid, toks)
        except vo.CapacityError:
            assert need > 0
            assert self._snapshot() == before
            return
        assert cached % self.bs == 0 and cached < len(toks)
        table = self._table(sid)
        for i in range(cached // self.bs):
            assert self.content.get(table[i]) == tuple(toks[:(i + 1) * self.bs])
        if not self.caching:
            assert cached == 0
        self.seqs[sid] = toks
        self._record_full_blocks(sid)

    @precondition(lambda self: self.seqs)
    @rule(data=st.data())
    def append(self, data):
        s = data.draw(st.sampled_from(sorted(self.seqs)))
        tok = data.draw(st.integers(0, 2))
        others = set()
        for o in self.seqs:
            if o != s:
                others.update(self._table(o))
        before = self._snapshot()
        try:
            slot, copy = self.bm.append_token(s, tok)
        except vo.CapacityError:
            assert self.bm.available() == 0
            assert self._snapshot() == before
            return
        pos = len(self.seqs[s])
        table = self._table(s)
        assert slot == table[pos // self.bs] * self.bs + pos % self.bs
        if copy is not None:
            src, dst = copy
            assert src in others and dst not in others and dst == table[pos // self.bs]
            assert pos % self.bs != 0
        self.seqs[s] = self.seqs[s] + [tok]
        self._record_full_blocks(s)

    @precondition(lambda self: self.seqs)
    @rule(data=st.data())
    def fork(self, data):
        s = data.draw(st.sampled_from(sorted(self.seqs)))
        c = self.next_id
        self.next_id += 1
        self.bm.fork(s, c)
        assert self._table(c) == self._table(s)
        self.seqs[c] = list(self.seqs[s])

    @precondition(lambda self: self.seqs)
    @rule(data=st.data())
    def free(self, data):
        s = data.draw(st.sampled_from(sorted(self.seqs)))
        self.bm.free(s)
        del self.seqs[s]

    # -- invariants --------------------------------------------------------
    @invariant()
    def manager_invariants(self):
        if not hasattr(self, "bm"):
            return
        self.bm.check()
        for s, toks in self.seqs.items():
            assert len(self._table(s)) == -(-len(toks) // self.bs)
            assert self.bm.num_tokens(s) == len(toks)
        assert self.bm.available() == self.N - len(self._live_blocks())
        st_ = self.bm.stats()
        assert st_["sequences"] == len(self.seqs)
        assert st_["free_blocks"] + st_["cached_idle_blocks"] == self.bm.available()


TestBlockManagerStateMachine = BlockManagerMachine.TestCase
TestBlockManagerStateMachine.settings = settings(
    max_examples=150, stateful_step_count=40, deadline=None,
    suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])


class CollidingHashMachine(BlockManagerMachine):
    unchained = True


TestBlockManagerCollidingHashes = CollidingHashMachine.TestCase
TestBlockManagerCollidingHashes.settings = TestBlockManagerStateMachine.settings


def test_prefix_hit_needs_the_same_verified_prefix():
    """A cached block is reused only after the very block the lookup accepted
    before it.  With the unchained-hash test hook a block hashes its own
    tokens only, so block T after prefix A and block T after prefix B
    collide: the prompt B + T finds sequence 1's T block (computed after A)
    and must not take it; A + T still hits both blocks."""
    bm = vo.BlockManager(32, 4)
    bm.test_unchained_hash(True)
    A, B, T = [1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]
    assert bm.add_sequence(1, A + T + [0]) == 0
    assert bm.add_sequence(2, B + [0]) == 0
    assert bm.add_sequence(3, B + T + [0]) == 4
    assert bm.block_table(3)[0] == bm.block_table(2)[0]
    assert bm.block_table(3)[1] != bm.block_table(1)[1]
    assert bm.add_sequence(4, T + [0]) == 0          # T was cached at position 1, not 0
    assert bm.add_sequence(5, A + T + [7]) == 8
    assert list(bm.block_table(5)[:2]) == list(bm.block_table(1)[:2])
    bm.check()


def test_duplicate_prompt_then_appends_stay_reachable():
    """The same prompt twice: the second copy's last-token block duplicates
    the first's cached block (first writer wins), so the cache's block stands
    for it in its verified chain.  The blocks it fills afterwards are
    registered after that block, so a later prompt with the second copy's
    tokens hits all of them; and a block whose predecessor has no verified
    link is not registered at all (it could never be hit, and would only hold
    a hash another sequence's valid block needs)."""
    bm = vo.BlockManager(64, 4)
    P = list(range(12))                              # 3 full blocks
    assert bm.add_sequence(1, P) == 0
    assert bm.add_sequence(2, P) == 8                # not the last token's block
    for t in [20, 21, 22, 23]:                       # fills block 3 of sequence 2 only
        bm.append_token(2, t)
    assert bm.add_sequence(3, P + [20, 21, 22, 23, 5]) == 16
    assert list(bm.block_table(3)[:4]) == [bm.block_table(1)[0], bm.block_table(1)[1],
                                           bm.block_table(1)[2], bm.block_table(2)[3]]
    for t in [30, 31, 32, 33]:                       # both fill block 3 alike
        bm.append_token(1, t)
    assert bm.add_sequence(4, P + [30, 31, 32, 33, 9]) == 16
    assert bm.block_table(4)[3] == bm.block_table(1)[3]
    bm.check()
    # Unchained hashes: sequence 6's block [9, 9, 9, 9] collides with the
    # cache's entry from sequence 5 (after another prefix), so its chain
    # breaks there, and its later block is not registered.
    bm = vo.BlockManager(64, 4)
    bm.test_unchained_hash(True)
    assert bm.add_sequence(5, [1, 1, 1, 1, 9, 9, 9, 9, 0]) == 0
    assert bm.add_sequence(6, [2, 2, 2, 2, 9, 9, 9, 9, 7, 7, 7, 7, 0]) == 0
    assert bm.add_sequence(7, [3, 3, 3, 3, 7, 7, 7, 7, 0]) == 0   # [7]*4 was not registered
    assert bm.add_sequence(8, [2, 2, 2, 2, 9, 9, 9, 9, 7, 7, 7, 7, 1]) == 4
    # so the hash of [7]*4 was free for sequence 7's own block, which a prompt
    # with sequence 7's prefix now hits
    assert bm.add_sequence(9, [3, 3, 3, 3, 7, 7, 7, 7, 2]) == 8
    with pytest.raises(vo.InvalidArgument):
        bm.test_unchained_hash(False)                # only before the first sequence
    bm.check()


def test_shared_prefix_blocks_and_last_token_block():
    """64 prompts with a common 4096-token prefix (cfg5's shape at block 16)
    share 256 blocks; a prompt that is exactly the cached prefix still gets
    its own last block, whose token the step must compute."""
    bm = vo.BlockManager(2000, 16)
    prefix = list(range(4096))
    assert bm.add_sequence(0, prefix + [1, 2, 3]) == 0
    for s in range(1, 64):
        assert bm.add_sequence(s, prefix + [s] * (s % 40 + 1)) == 4096
    t0 = bm.block_table(0)
    for s in range(1, 64):
        assert np.array_equal(bm.block_table(s)[:256], t0[:256])
    assert bm.add_sequence(100, prefix) == 4096 - 16
    assert bm.block_table(100)[255] != t0[255]
    bm.check()


def test_freed_prefix_stays_cached_until_evicted():
    bm = vo.BlockManager(8, 4)
    bm.add_sequence(1, list(range(12)) + [99])
    bm.free(1)
    assert bm.available() == 8
    assert bm.add_sequence(2, list(range(12)) + [5]) == 12   # hit on idle cached blocks
    bm.free(2)
    bm.add_sequence(3, [7] * 32)                              # needs all 8: evicts the cache
    assert bm.stats()["evictions"] >= 3
    bm.free(3)
    assert bm.add_sequence(4, list(range(12)) + [5]) == 0
    bm.check()


def test_fork_copy_on_write_and_capacity():
    bm = vo.BlockManager(3, 4)
    bm.add_sequence(1, [1, 2, 3, 4, 5, 6])
    bm.fork(1, 2)
    slot, copy = bm.append_token(2, 9)        # block 1 is shared: copied
    assert copy is not None and copy[0] == bm.block_table(1)[1]
    assert slot == bm.block_table(2)[1] * 4 + 2
    slot, copy = bm.append_token(1, 8)        # no longer shared
    assert copy is None
    with pytest.raises(vo.CapacityError):
        bm.add_sequence(3, [1] * 9)
    bm.check()


def test_errors():
    bm = vo.BlockManager(4, 4)
    bm.add_sequence(1, [1])
    with pytest.raises(vo.InvalidArgument):
        bm.add_sequence(1, [2])
    with pytest.raises(vo.InvalidArgument):
        bm.append_token(7, 1)
    with pytest.raises(vo.InvalidArgument):
        bm.free(7)
    with pytest.raises(vo.ShapeError):
        vo.BlockManager(0, 4)
