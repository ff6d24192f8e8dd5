"""The batch scheduler (kh_sched_run) against the oracle's golden outputs of each case, and against
one batch plan per case: each sequence's result does not depend on its batch-mates, plan length or
chunk (the batch/single identity of test_gpu_models), so the scheduled outputs equal the batch
plan's bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from kleinhirn_amd import configs
from kleinhirn_amd.backend import HipBackend, KhError
from kleinhirn_amd.scheduler import BatchScheduler
from tests.helpers import decision_parity, hip_outputs
from tests.test_gpu_models import case_and_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("key", ["c2", "c5"])
def test_scheduled_outputs_equal_the_batch_plan(key):
    case, ref = case_and_oracle(key)
    want = hip_outputs(case, f16=True)
    W = configs.storage(case.weights, True)
    be = HipBackend(W)
    be.set_words(W["embeddings.word.weight"])
    sch = BatchScheduler(be, case.spec, case.head, True, lengths=(128, case.length), batch=4, copies=2)
    n = [len(x) for x in case.ids]
    out, st = sch.run(case.ids)
    print(key, st)
    d = decision_parity(ref, out)
    assert d["mismatched"] == 0 and d["delta"] <= 2e-2, d
    assert np.array_equal(out, want)
    assert st["sequences"] == len(n) and st["tokens"] == sum(n) and st["chunks"] >= -(-len(n) // 4)
    budget = max(n) + 10
    out2, st2 = sch.run(case.ids, token_budget=budget)
    assert np.array_equal(out2, want)
    assert st2["chunks"] > st["chunks"]
    # input order is kept whatever the length order
    rev, _ = sch.run(case.ids[::-1])
    assert np.array_equal(rev, want[::-1])
    with pytest.raises(KhError, match="exceeds the longest plan"):
        sch.run([np.ones(case.length + 1, np.int32)])
    sch.destroy()
    be.dispose()
