"""Host data pipeline (libsft_pipeline.so): the properties the reference's own
pipeline tests fix (src/rust/pipeline.rs:1360-1549) -- a round trip without
shuffle returns every entry in order, the shuffle is a seed-dependent
permutation, the skip filter drops the known entries, rank shards are
disjoint and cover the data -- plus the random stream against the published
xoshiro256++ / SplitMix64 test vectors, each skip rule alone, the chunk scan
and its sidecar cache, several readers, cyclic mode and error reporting."""

import os

import numpy as np
import pytest

from sft_amd import pipeline as pl
from sft_amd import positions


def _entries(n, seed=0, **kw):
    boards, stm = positions.random_positions(n, seed=seed)
    g = np.random.default_rng(seed + 100)
    e = pl.make_entries(boards, stm, score=g.integers(-3000, 3000, n), result=g.integers(-1, 2, n),
                        ply=g.integers(0, 200, n))
    for k, v in kw.items():
        e[k] = v
    return e


def _key(boards, stm, score):
    """Entry identity as a batch shows it: the board, side to move and score."""
    return [bytes(b) + bytes([s]) + int(sc).to_bytes(4, "little", signed=True)
            for b, s, sc in zip(boards, stm, score)]


def _collect(stream):
    keys, outcome = [], []
    for batch in stream:
        keys += _key(batch.boards, batch.side_to_move, batch.score.astype(np.int64))
        outcome += batch.outcome.tolist()
        assert batch.size <= stream.batch_size
        batch.release()
    stream.close()
    return keys, outcome


def _expected(e):
    return _key(e["board"], e["side_to_move"], e["score"])


def test_random_stream_matches_published_vectors():
    # xoshiro256++ from state (1, 2, 3, 4): the reference implementation's first outputs
    want = [41943041, 58720359, 3588806011781223, 3591011842654386, 9228616714210784205, 9973669472204895162,
            14011001112246962877, 12406186145184390807, 15849039046786891736, 10450023813501588000]
    assert pl.rng_u64(10, state=np.array([1, 2, 3, 4], np.uint64)).tolist() == want
    # seeding from a u64 fills the state with SplitMix64 outputs (seed 1234567's published sequence)
    splitmix = np.array([6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431],
                        np.uint64)
    assert np.array_equal(pl.rng_u64(20, seed=1234567), pl.rng_u64(20, state=splitmix))


def test_round_trip_without_shuffle(tmp_path):
    e = _entries(1000, seed=1)
    path = str(tmp_path / "a.sftpos")
    pl.write_entries(path, e, entries_per_chunk=1000)
    keys, outcome = _collect(pl.BatchStream([path], 7, reader_threads=1, shuffle_buffer_entries=0, seed=0))
    assert keys == _expected(e)  # every entry once, in order (one chunk, one reader)
    assert np.array_equal(np.array(outcome, np.float32), (e["result"].astype(np.float32) + 1) / 2)


def test_shuffle_is_a_permutation_and_changes_with_seed(tmp_path):
    e = _entries(24, seed=2)
    path = str(tmp_path / "s.sftpos")
    pl.write_entries(path, e)
    original = _expected(e)
    orders = []
    for seed in (1, 7):
        keys, _ = _collect(pl.BatchStream([path], 4, reader_threads=1, shuffle_buffer_entries=8, seed=seed))
        assert sorted(keys) == sorted(original)
        orders.append(keys)
    assert any(o != original for o in orders)
    assert orders[0] != orders[1]
    # the same seed gives the same order
    again, _ = _collect(pl.BatchStream([path], 4, reader_threads=1, shuffle_buffer_entries=8, seed=7))
    assert again == orders[1]


def test_skip_filter_removes_known_entries(tmp_path):
    # the reference's four entries (pipeline.rs:1446-1511)
    fen = lambda f: positions.board_from_fen(f)  # noqa: E731
    b0, s0 = fen("4k3/8/8/8/8/8/8/4K3 w - - 0 1")
    b2, s2 = fen("4k3/8/8/8/8/8/4p3/4K3 w - - 0 1")
    e1, e2, d1 = 4, 12, 3
    boards = np.stack([b0, b0, b2, b0])
    e = pl.make_entries(boards, [s0, s0, s2, s0], score=[pl.VALUE_NONE, 50, 50, 200], ply=[10, 1, 10, 20],
                        result=[0, 0, 0, 1], move_from=[e1] * 4, move_to=[e2, e2, e2, d1])
    path = str(tmp_path / "k.sftpos")
    pl.write_entries(path, e)
    keys, _ = _collect(pl.BatchStream([path], 8, reader_threads=1, shuffle_buffer_entries=0, filtered=True,
                                      early_fen_skipping=4, pc_y1=1.0, pc_y2=1.0, pc_y3=1.0))
    assert not set(_expected(e[:3])) & set(keys)
    skip = pl.skip_filter(e, filtered=True, early_fen_skipping=4, pc_y1=1.0, pc_y2=1.0, pc_y3=1.0)
    assert skip[:3].all()


def test_each_skip_rule():
    fen = lambda f: positions.board_from_fen(f)  # noqa: E731
    quiet, w = fen("4k3/8/8/8/8/8/8/R3K3 w - - 0 1")
    check, _ = fen("4k3/8/8/8/8/8/8/4K2r w - - 0 1")       # rook on h1 checks the white king on e1
    pawn_check, _ = fen("4k3/8/8/8/8/8/3p4/4K3 w - - 0 1")  # black pawn on d2 checks e1
    capture, _ = fen("4k3/8/8/8/8/8/8/R3K2r w - - 0 1")
    # rules checked on entries they must skip whatever the piece-count rule draws
    keep = dict(pc_y1=1.0, pc_y2=1.0, pc_y3=1.0)
    e = pl.make_entries(np.stack([quiet, check, pawn_check, quiet]), [w] * 4, score=100, ply=30,
                        move_from=[0, 0, 0, 0], move_to=[8, 8, 8, 8])
    e["move_to"][3] = 7  # a1 -> h1 onto the black rook: a capture
    e["board"][3] = capture
    filt = pl.skip_filter(e, filtered=True, **keep)
    assert filt[1] and filt[2] and filt[3]  # in check (rook, pawn), capture
    assert not pl.skip_filter(e).any()  # no rule enabled: nothing skipped
    early = pl.make_entries(np.stack([quiet] * 3), [w] * 3, ply=[3, 4, 5])
    assert pl.skip_filter(early, early_fen_skipping=4, **keep)[:2].all()
    none = pl.make_entries(np.stack([quiet] * 2), [w] * 2, score=[pl.VALUE_NONE, pl.VALUE_NONE])
    assert pl.skip_filter(none, early_fen_skipping=0, **keep).all()
    # random skipping with n = 3 skips 3/4 before the piece-count rule
    many = _entries(20000, seed=3)
    frac = pl.skip_filter(many, random_fen_skipping=3, seed=5).mean()
    assert 0.75 < frac < 1.0
    # material: |eval| < threshold skipped (kings + a rook = 1276 for the side with it)
    rook = pl.make_entries(np.stack([quiet] * 2), [0, 1], score=10, ply=50)
    assert pl.skip_filter(rook, simple_eval_skipping=2000, early_fen_skipping=0, **keep).all()


def test_piece_count_rule_follows_the_desired_distribution():
    """After the first 10000 entries the piece-count rule keeps counts in
    proportion to the desired weights (pipeline.rs:672-696): with weights
    y(0) = y(32) = 1, y(16) = 2, positions of 16 pieces are kept about twice as
    often as positions of 32 pieces would be relative to their frequency."""
    g = np.random.default_rng(9)
    n = 40000
    boards = np.full((n, 64), positions.EMPTY, np.uint8)
    counts = np.where(g.random(n) < 0.5, 16, 32)
    for i in range(n):
        sq = g.permutation(64)[:counts[i]]
        boards[i, sq] = g.integers(0, 10, counts[i])
    e = pl.make_entries(boards, 0, score=0, ply=100)
    skip = pl.skip_filter(e, early_fen_skipping=0, seed=1)  # enables the filter; every ply passes
    tail = slice(20000, None)
    k16 = (~skip[tail] & (counts[tail] == 16)).sum() / (counts[tail] == 16).sum()
    k32 = (~skip[tail] & (counts[tail] == 32)).sum() / (counts[tail] == 32).sum()
    assert 1.6 < k16 / k32 < 2.4, (k16, k32)


def test_rank_shards_are_disjoint_and_cover(tmp_path):
    files = []
    for i in range(2):
        p = str(tmp_path / f"r{i}.sftpos")
        pl.write_entries(p, _entries(6, seed=10 + i), entries_per_chunk=1)
        files.append(p)
    shards = []
    for rank in range(2):
        keys, _ = _collect(pl.BatchStream(files, 4, reader_threads=2, shuffle_buffer_entries=0, rank=rank,
                                          world_size=2, seed=3))
        shards.append(set(keys))
    assert not shards[0] & shards[1]
    every = set(_expected(_entries(6, seed=10))) | set(_expected(_entries(6, seed=11)))
    assert shards[0] | shards[1] == every


def test_many_readers_deliver_every_entry_once(tmp_path):
    e = _entries(5000, seed=4)
    path = str(tmp_path / "m.sftpos")
    pl.write_entries(path, e, entries_per_chunk=97)
    stream = pl.BatchStream([path], 256, reader_threads=6, shuffle_buffer_entries=300, seed=11, slab_count=3)
    keys, _ = _collect(stream)
    assert sorted(keys) == sorted(_expected(e))


def test_chunk_scan_and_sidecar_cache(tmp_path):
    e = _entries(250, seed=5)
    path = str(tmp_path / "c.sftpos")
    pl.write_entries(path, e, entries_per_chunk=100)
    off, cnt = pl.scan_chunks(path)
    assert cnt.tolist() == [100, 100, 50]
    assert off.tolist() == [8, 8 + 8 + 7200, 8 + 2 * (8 + 7200)]
    assert os.path.exists(path + ".chunks")
    assert pl.scan_chunks(path)[1].tolist() == [100, 100, 50]  # from the cache
    with open(path + ".chunks", "r+b") as f:  # a cache for another file size is ignored
        f.seek(8)
        f.write((123).to_bytes(8, "little"))
    assert pl.scan_chunks(path)[1].tolist() == [100, 100, 50]
    bad = str(tmp_path / "bad.sftpos")
    with open(bad, "wb") as f:
        f.write(b"XXXX" + (72).to_bytes(4, "little") + bytes(72))
    with pytest.raises(RuntimeError, match="bad chunk header"):
        pl.scan_chunks(bad)


def test_cyclic_stream_keeps_going(tmp_path):
    e = _entries(30, seed=6)
    path = str(tmp_path / "y.sftpos")
    pl.write_entries(path, e, entries_per_chunk=10)
    stream = pl.BatchStream([path], 16, reader_threads=2, shuffle_buffer_entries=0, cyclic=True, seed=1)
    seen = 0
    for _ in range(10):  # 160 entries from a 30-entry file
        b = stream.next_batch()
        assert b is not None and b.size == 16
        seen += b.size
        b.release()
    stream.close()
    assert seen == 160


def test_errors_are_reported():
    with pytest.raises(RuntimeError, match="cannot stat"):
        pl.BatchStream(["/nonexistent/file.sftpos"], 4)
    with pytest.raises(RuntimeError, match="rank must be less than world_size"):
        pl.BatchStream(["x"], 4, rank=2, world_size=2)
    with pytest.raises(RuntimeError, match="batch_size"):
        pl.BatchStream(["x"], 0)


def test_header_declares_the_binding_table():
    import re

    from conftest import ROOT

    text = open(os.path.join(ROOT, "include", "sft_pipeline.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    assert sorted(set(re.findall(r"\b(sft_\w+)\s*\(", text))) == sorted(pl.SIGNATURES)
    lib = pl.lib()
    for name in pl.SIGNATURES:
        assert hasattr(lib, name), name
