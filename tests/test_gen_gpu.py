"""GPU: the stream generator (gen_tokens / gen_set / gen_copies) makes the same bytes as the numpy generator."""

import numpy as np
import pytest

from ngram_amd import data
from ngram_amd.lib import Lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,train,query", [("c1", 300_000, 30_001), ("c3", 500_000, 200_001)])
def test_gpu_generator_matches_numpy(name, train, query):
    cfg = data.CONFIGS[name]
    zipf, tp, qp = data.make_plans(cfg, train, query)
    host_t = data.realize(tp, zipf)
    host_q = data.realize(qp, zipf, host_t)
    lib = Lib()
    gpu_t = data.realize_gpu(tp, zipf, lib)
    gpu_q = data.realize_gpu(qp, zipf, lib, source=gpu_t)
    assert np.array_equal(gpu_t.cpu().numpy().view(np.uint16), host_t)
    assert np.array_equal(gpu_q.cpu().numpy().view(np.uint16), host_q)
    assert len(tp.copies) and len(qp.copies)
