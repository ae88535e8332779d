"""Host serving core (scheduler + block manager with prefix caching) on the CPU.

The reference ships no tests for engine/scheduler.cpp or engine/block_manager.cpp; these pin the
behaviour its code fixes by hand-computed scenarios (chunking, budget, groups, LRF reuse, prefix
hits, preemption) and by invariants over seeded random workloads."""
import numpy as np
import pytest

from cppvllm_amd.engine_core import GROUP_CONT, GROUP_DECODE, GROUP_FRESH, EngineBusy, EngineCore


def run_to_end(core, token_fn=lambda sid, step: 7, max_steps=100000):
    """Drive the core with a fake sampler; returns the list of batches seen."""
    seen = []
    step = 0
    while not core.is_finished():
        b = core.schedule()
        assert b is not None
        seen.append(b)
        core.postprocess([token_fn(int(s), step) if smp else -1 for s, smp in zip(b.seq_ids, b.samples)])
        step += 1
        assert step < max_steps
    return seen


def groups_of(b):
    g = np.zeros(b.num_seqs, dtype=int)
    for k in range(3):
        g[b.group_start[k]:b.group_start[k + 1]] = k
    return g


def test_single_request_prefill_then_decode():
    core = EngineCore(block_size=16, num_blocks=64)
    prompt = list(range(100, 140))
    rid = core.add_request(prompt, max_tokens=3)
    b = core.schedule()
    assert b.num_seqs == 1 and b.num_tokens == 40
    assert list(b.tokens) == prompt and list(b.positions) == list(range(40))
    assert b.kv_lens[0] == 40 and b.samples[0]
    assert b.group_start == (0, 0, 1, 1)               # a fresh prefill
    assert list(b.block_tables[0]) == core.block_table(rid)[:3]
    core.postprocess([11])
    b = core.schedule()                                 # decode: the sampled token at position 40
    assert list(b.tokens) == [11] and list(b.positions) == [40] and b.kv_lens[0] == 41
    assert b.group_start == (0, 1, 1, 1)
    core.postprocess([12])
    b = core.schedule()
    assert list(b.tokens) == [12] and b.kv_lens[0] == 42
    core.postprocess([13])
    assert core.is_finished()
    assert core.take_finished() == {rid: [11, 12, 13]}
    assert core.stats().free_blocks == 64


def test_chunked_prefill_and_budget():
    core = EngineCore(block_size=16, num_blocks=64, max_chunk_tokens=16, max_num_batched_tokens=24)
    a = core.add_request(list(range(40)), max_tokens=1)
    b_ = core.add_request(list(range(1000, 1030)), max_tokens=1)
    b = core.schedule()              # a: 16 (chunk cap), b: 8 (budget left)
    assert list(b.seq_ids) == [a, b_] and list(np.diff(b.cu_seqlens)) == [16, 8]
    assert not b.samples.any()
    assert list(groups_of(b)) == [GROUP_FRESH, GROUP_FRESH]
    core.postprocess([-1, -1])
    b = core.schedule()              # a: next 16 (cached 16 -> continuation), b: 8 more
    assert list(np.diff(b.cu_seqlens)) == [16, 8]
    assert list(b.positions[:2]) == [16, 17] and b.positions[16] == 8
    assert list(groups_of(b)) == [GROUP_CONT, GROUP_CONT]
    assert list(b.kv_lens) == [32, 16]
    core.postprocess([-1, -1])
    b = core.schedule()              # a: last 8 (samples), b: 14 -> 16 cap but 16 budget left
    assert list(np.diff(b.cu_seqlens)) == [8, 14] and list(b.samples) == [True, True]
    core.postprocess([5, 6])
    assert core.is_finished()
    assert core.take_finished() == {a: [5], b_: [6]}


def test_max_num_seqs():
    core = EngineCore(block_size=16, num_blocks=64, max_num_seqs=2)
    ids = [core.add_request([1, 2, 3], max_tokens=2) for _ in range(3)]
    b = core.schedule()
    assert list(b.seq_ids) == ids[:2]
    core.postprocess([9, 9])
    b = core.schedule()              # the third waits until a slot frees
    assert list(b.seq_ids) == ids[:2]
    core.postprocess([9, 9])
    b = core.schedule()
    assert list(b.seq_ids) == [ids[2]]


def test_prefix_cache_hits_and_sharing():
    bs = 16
    core = EngineCore(block_size=bs, num_blocks=32)
    shared = list(range(500, 548))                      # 3 full blocks
    a = core.add_request(shared + [1, 2], max_tokens=4)
    core.postprocess([7] * core.schedule().num_seqs)    # prefill a (commits its 3 full blocks)
    ta = core.block_table(a)
    b_ = core.add_request(shared + [9], max_tokens=1)
    b = core.schedule()                                 # a decodes; b hits 3 blocks, computes 1 token
    assert core.stats().prefix_hit_tokens == 48
    tb = core.block_table(b_)
    assert tb[:3] == ta[:3] and tb[3] not in ta
    for blk in ta[:3]:
        assert core.ref_count(blk) == 2
    j = list(b.seq_ids).index(b_)
    assert b.kv_lens[j] == 49 and b.cu_seqlens[j + 1] - b.cu_seqlens[j] == 1 and b.positions[b.cu_seqlens[j]] == 48
    assert groups_of(b)[j] == GROUP_DECODE              # one new token on a cached context
    # both rows report their 3 shared leading blocks (for the attention plan's cache-resident reads)
    assert list(b.shared_blocks) == [3, 3]
    core.postprocess([7 if s else -1 for s in b.samples])
    run_to_end(core)
    assert core.stats().free_blocks == 32


def test_prompt_ending_on_a_block_boundary_recomputes_its_last_block():
    core = EngineCore(block_size=16, num_blocks=32)
    p = list(range(32))
    core.add_request(p, max_tokens=1)
    run_to_end(core)
    core.add_request(p, max_tokens=1)
    b = core.schedule()
    # (32 - 1) // 16 = 1 cacheable block: 16 tokens are recomputed so the step samples
    assert b.num_tokens == 16 and b.positions[0] == 16 and b.samples[0]


def test_lrf_reuse_order():
    core = EngineCore(block_size=16, num_blocks=8)
    a = core.add_request(list(range(40)), max_tokens=1)       # 3 blocks: 0, 1, 2
    core.schedule()
    assert core.block_table(a) == [0, 1, 2]
    core.postprocess([1])                                     # finished: freed tail first 2, 1, 0
    b = core.add_request(list(range(1000, 1100)), max_tokens=1)   # 7 blocks from the free list
    core.schedule()
    # fresh blocks come from the head: the never-used 3..7, then the least recently freed 2, 1
    assert core.block_table(b) == [3, 4, 5, 6, 7, 2, 1]


def test_preemption_by_recompute():
    bs = 16
    core = EngineCore(block_size=bs, num_blocks=6)
    a = core.add_request(list(range(30)), max_tokens=40)      # needs up to 5 blocks
    b_ = core.add_request(list(range(100, 130)), max_tokens=30)
    seen = run_to_end(core, token_fn=lambda s, st: 3)
    st = core.stats()
    assert st.preemptions >= 1
    out = core.take_finished()
    assert len(out[a]) == 40 and len(out[b_]) == 30
    assert st.free_blocks == 6
    # after a preemption the victim's whole context is recomputed as a prefill
    assert any(b.num_tokens > 1 and b.num_seqs == 1 for b in seen[2:])


def test_errors():
    core = EngineCore(block_size=16, num_blocks=4)
    with pytest.raises(ValueError):
        core.add_request(list(range(60)), max_tokens=10)      # 70 tokens > 4 blocks
    with pytest.raises(RuntimeError):
        core.postprocess([])                                  # nothing scheduled
    with pytest.raises(ValueError):
        core.add_request([], max_tokens=1)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_workload_invariants(seed):
    rng = np.random.default_rng(seed)
    bs = 16
    nblocks = 200
    core = EngineCore(block_size=bs, num_blocks=nblocks, max_num_batched_tokens=256, max_num_seqs=12,
                      max_chunk_tokens=64)
    base = rng.integers(0, 50, 64).tolist()              # common prefix for some requests
    reqs = {}
    for _ in range(30):
        n = int(rng.integers(1, 150))
        p = (base[:int(rng.integers(0, 64))] + rng.integers(0, 50, n).tolist()) if rng.random() < 0.5 else \
            rng.integers(0, 50, n).tolist()
        m = int(rng.integers(1, 60))
        reqs[core.add_request(p, max_tokens=m)] = (p, m)
    ctx = {rid: list(p) for rid, (p, m) in reqs.items()}   # what each request's tokens must be
    step = 0
    while not core.is_finished():
        b = core.schedule()
        T = b.num_tokens
        assert T <= 256 and b.num_seqs <= 12
        used = set()
        for j in range(b.num_seqs):
            rid = int(b.seq_ids[j])
            t0, t1 = b.cu_seqlens[j], b.cu_seqlens[j + 1]
            assert 0 < t1 - t0 <= 64
            pos = b.positions[t0:t1]
            assert list(pos) == list(range(pos[0], pos[0] + (t1 - t0)))
            assert b.kv_lens[j] == pos[-1] + 1
            assert list(b.tokens[t0:t1]) == ctx[rid][pos[0]:pos[-1] + 1]
            nb = -(-b.kv_lens[j] // bs)
            row = b.block_tables[j]
            assert (row[:nb] >= 0).all() and (row[nb:] == -1).all()
            # blocks written this step (positions' blocks) belong to this sequence alone
            for blk in set(row[pos // bs].tolist()):
                assert blk not in used
                used.add(blk)
            g = groups_of(b)[j]
            if g == GROUP_DECODE:
                assert t1 - t0 == 1 and pos[0] > 0
            elif g == GROUP_FRESH:
                assert pos[0] == 0 and t1 - t0 > 1
        sampled = []
        for j in range(b.num_seqs):
            if b.samples[j]:
                tok = int(rng.integers(0, 50))
                ctx[int(b.seq_ids[j])].append(tok)
                sampled.append(tok)
            else:
                sampled.append(-1)
        core.postprocess(sampled)
        step += 1
        assert step < 20000
    out = core.take_finished()
    assert set(out) == set(reqs)
    for rid, (p, m) in reqs.items():
        assert len(out[rid]) == m
        assert out[rid] == ctx[rid][len(p):]
    assert core.stats().free_blocks == nblocks


# ---- two-deep launch ring (engine/llm_engine.cpp:70-113) -------------------------------------------------
V = 997


def fake_model(b, prev_sampled):
    """Next token of every sampling row from its context's last token and position; tokens the
    previous step is sampling (feed_src >= 0) are read from that step's samples, as the device
    feed does."""
    toks = b.tokens.copy()
    feed = b.feed_src
    if feed is not None and (feed >= 0).any():
        assert prev_sampled is not None
        toks[feed >= 0] = prev_sampled[feed[feed >= 0]]
    assert (toks >= 0).all()
    out = np.full(b.num_seqs, -1, dtype=np.int64)
    for j in range(b.num_seqs):
        if b.samples[j]:
            t = b.cu_seqlens[j + 1] - 1
            out[j] = (int(toks[t]) * 31 + int(b.positions[t]) * 7 + 3) % V
    return out


def drive(core, depth):
    """Run to completion keeping up to `depth` steps outstanding; returns the step count."""
    ring = []                 # (batch, sampled) of outstanding steps, oldest first
    steps = 0
    while not core.is_finished():
        if len(ring) < depth:
            try:
                b = core.schedule()
            except EngineBusy:
                b = "busy"
            if b is not None and b != "busy":
                prev = ring[-1][1] if ring else None
                ring.append((b, fake_model(b, prev)))
                steps += 1
                assert steps < 20000
                if len(ring) < depth:
                    continue
            elif b is None and not ring:
                break
        _, s = ring.pop(0)
        core.postprocess(s)
    while ring:
        core.postprocess(ring.pop(0)[1])
    return steps


def make_core(**kw):
    return EngineCore(block_size=16, num_blocks=kw.pop("num_blocks", 400), max_num_batched_tokens=256,
                      max_num_seqs=kw.pop("max_num_seqs", 16), max_chunk_tokens=64, **kw)


def workload(core, seed, n=40, eos=False):
    rng = np.random.default_rng(seed)
    ids = []
    for _ in range(n):
        p = rng.integers(0, V, int(rng.integers(1, 120))).tolist()
        ids.append(core.add_request(p, max_tokens=int(rng.integers(1, 50)), ignore_eos=not eos))
    return ids


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("eos", [False, True])
def test_ring_matches_synchronous_steps(seed, eos):
    outs = []
    for depth in (1, 2):
        core = make_core(eos_token_id=5 if eos else -1)
        ids = workload(core, seed, eos=eos)
        drive(core, depth)
        got = core.take_finished()
        outs.append([got[i] for i in ids])
        assert core.stats().free_blocks == 400
        assert core.outstanding() == 0
    assert outs[0] == outs[1]
    if eos:   # some request did stop at the EOS token
        assert any(o and o[-1] == 5 for o in outs[1])


def test_ring_feeds_the_previous_steps_samples():
    core = make_core()
    rid = core.add_request([1, 2, 3], max_tokens=4)
    b0 = core.schedule()                         # prefill, samples token 3's successor
    assert b0.samples[0] and (b0.feed_src == -1).all()
    b1 = core.schedule()                         # decode of the token b0 is still sampling
    assert list(b1.tokens) == [-1] and list(b1.feed_src) == [0] and list(b1.positions) == [3]
    with pytest.raises(RuntimeError):
        core.schedule()                          # two steps outstanding
    assert core.outstanding() == 2
    core.postprocess([40])
    b2 = core.schedule()
    assert list(b2.feed_src) == [0] and list(b2.positions) == [4]
    core.postprocess([41])
    core.postprocess([42])
    b3 = core.schedule()                         # synchronous again: the token is known
    assert list(b3.tokens) == [42] and list(b3.feed_src) == [-1]
    core.postprocess([43])
    assert core.is_finished() and core.take_finished() == {rid: [40, 41, 42, 43]}


def test_ring_does_not_schedule_past_max_tokens():
    core = make_core()
    rid = core.add_request([9, 9], max_tokens=1)
    core.schedule()                              # its only token is being sampled
    with pytest.raises(EngineBusy):
        core.schedule()                          # nothing else to run until that step retires
    core.postprocess([77])
    assert core.is_finished() and core.take_finished() == {rid: [77]}


def test_ring_defers_preemption_until_drained():
    core = EngineCore(block_size=16, num_blocks=6, max_num_batched_tokens=256, max_num_seqs=4)
    a = core.add_request(list(range(40)), max_tokens=40)     # 3 blocks now, 5 at the end
    b = core.add_request(list(range(100, 130)), max_tokens=40)
    steps = drive(core, 2)
    out = core.take_finished()
    assert len(out[a]) == 40 and len(out[b]) == 40
    assert core.stats().preemptions >= 1 and core.stats().free_blocks == 6
    assert steps > 0
