"""Host pipeline -> GPU: batches of positions from the pipeline's pinned slabs,
copied to the device and encoded there, equal the oracle's encoding of the
same entries (index rows, side to move, buckets), with outcome and score."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, host
from oracle import feature_oracle as fo
from sft_amd import pipeline as pl
from sft_amd import positions

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("pin", [True, False])
def test_pipeline_batches_encode_on_the_gpu(tmp_path, pin):
    announce(f"pipeline -> GPU encode pin={pin}")
    boards, stm = positions.random_positions(3000, seed=21)
    g = np.random.default_rng(22)
    e = pl.make_entries(boards, stm, score=g.integers(-3000, 3000, 3000), result=g.integers(-1, 2, 3000), ply=50)
    path = str(tmp_path / "p.sftpos")
    pl.write_entries(path, e, entries_per_chunk=500)
    stream = pl.BatchStream([path], 1024, reader_threads=3, shuffle_buffer_entries=256, seed=5, pin_memory=pin)
    seen = 0
    for batch in stream:
        us, white, black, outcome, score, psqt, ls = batch.to_device(DEV, "Full_Threats+HalfKAv2_hm")
        torch.cuda.synchronize()
        b, s = batch.boards.copy(), batch.side_to_move.copy()
        ref = fo.encode(b, s, ["Full_Threats", "HalfKAv2_hm"])
        assert np.array_equal(host(white), ref["white"]) and np.array_equal(host(black), ref["black"])
        assert np.array_equal(host(us).reshape(-1), ref["us"])
        assert np.array_equal(host(psqt), ref["psqt"]) and np.array_equal(host(ls), ref["psqt"])
        assert np.array_equal(host(outcome).reshape(-1), batch.outcome)
        assert np.array_equal(host(score).reshape(-1), batch.score)
        seen += batch.size
        batch.release()
    stream.close()
    assert seen == 3000
