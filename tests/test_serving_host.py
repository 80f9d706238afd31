"""Host logic of the continuous-batch backend (no GPU): the contract passes the reference's own
admission rules (shard/continuous_batch.py:18-48, restated here as the expected answers), and advance_batch
keeps the per-job semantics RingPool.execute_batch_step / ContinuousRingWorker rely on
(shard/ring_pool.py:627-700, shard/continuous_batch.py:98-156).  The model is a deterministic fake
with the GptOssModel.step signature."""
import hashlib
import json

import pytest

from flyai_amd.serving import CONTRACT_KEYS, GptOssBatchBackend, contract_digest
from flyai_amd.weights import GptOssShape

V = 97


class FakeModel:
    """next token = f(every token fed so far to the slot), fed chunk by chunk at explicit starts."""

    def __init__(self, max_jobs=4, max_context=64, max_step_rows=64):
        self.shape = GptOssShape(n_experts=8)
        self.vocab, self.n_layers = V, 2
        self.max_jobs, self.max_context, self.max_step_rows = max_jobs, max_context, max_step_rows
        self.per_job_state_bytes = 1000
        self.hist = {}
        self.steps = []

    @staticmethod
    def next_token(seq):
        return int(hashlib.sha256(json.dumps(seq).encode()).hexdigest(), 16) % V

    def step(self, chunks, starts, slots, pick):
        self.steps.append([len(c) for c in chunks])
        assert sum(len(c) for c in chunks) <= self.max_step_rows
        out = []
        for c, s, sl, p in zip(chunks, starts, slots, pick):
            h = self.hist.setdefault(sl, [])
            assert len(h) >= s, "a chunk may not skip positions"
            del h[s:]
            h.extend(c)
            out.append(self.next_token(h) if p else None)
        return out


class JobCancelled(Exception):
    pass


class RingUnavailable(Exception):
    pass


class Job:
    def __init__(self, jid, prompt, max_new, tokens=()):
        self.id, self.payload, self.max_new = jid, {"ids": list(prompt)}, max_new
        self.prompt_tokens = len(prompt)
        self.tokens = list(tokens)
        self.cancelled = False

    def checkpoint(self):
        return list(self.tokens)


def backend(model=None, **kw):
    args = dict(model_id="gpt-oss-test", cohort_id="c1", tokenize=lambda p: p["ids"], max_prompt_tokens=32,
                max_new_tokens=16, prefill_chunk_tokens=4, source_sha256="a" * 64)
    args.update(kw)
    return GptOssBatchBackend(model or FakeModel(), **args)


def reference_contract_checks(value, model_id, cohort_id):
    """The admission rules of backend_contract (shard/continuous_batch.py:18-48)."""
    assert isinstance(value, dict) and set(value) == set(CONTRACT_KEYS) and value["schema"] == "shard-token-batch/1"
    assert value["model_id"] == model_id and value["cohort_id"] == cohort_id
    assert value["cancellation"] == "per_job" and isinstance(value["numerical_contract"], str) and value["numerical_contract"]
    for name in ("source_sha256", "runtime_config_sha256"):
        assert isinstance(value[name], str) and len(value[name]) == 64 and all(c in "0123456789abcdef" for c in value[name])
    for name in ("max_jobs", "max_step_tokens", "max_prompt_tokens", "max_new_tokens", "max_context_tokens",
                 "per_job_state_bytes", "reserved_state_bytes", "prefill_chunk_tokens"):
        assert type(value[name]) is int and 1 <= value[name] < 2 ** 63
    assert value["max_jobs"] <= 32 and value["max_step_tokens"] <= 64
    assert value["prefill_chunk_tokens"] <= value["max_prompt_tokens"]
    assert value["per_job_state_bytes"] * value["max_jobs"] <= value["reserved_state_bytes"]
    assert value["max_prompt_tokens"] < value["max_context_tokens"] and value["max_new_tokens"] <= value["max_context_tokens"]
    json.loads(json.dumps(value, allow_nan=False))


def run_worker(be, jobs, max_step_tokens=1, cancel=(), limit=200):
    """A minimal ContinuousRingWorker loop: advance until every job has an outcome."""
    done = {}
    active = list(jobs)
    per_call = []
    for _ in range(limit):
        if not active:
            break
        counts = {j.id: 0 for j in active}

        def emit_for(job):
            def emit(tok):
                if job.cancelled:
                    raise JobCancelled("job cancelled")
                counts[job.id] += 1
                assert counts[job.id] <= max_step_tokens, "backend exceeded its bounded token step"
                job.tokens.append(tok)
            return emit

        def check_for(job):
            def check():
                if job.id in cancel:
                    job.cancelled = True
                    raise JobCancelled("job cancelled")
            return check

        out = be.advance_batch(active, emit={j.id: emit_for(j) for j in active},
                               cancel_check={j.id: check_for(j) for j in active}, max_step_tokens=max_step_tokens)
        assert set(out) == {j.id for j in active}
        per_call.append(dict(counts))
        for j in list(active):
            if out[j.id] is not None:
                done[j.id] = out[j.id]
                be.release_batch_job(j.id)
                active.remove(j)
    assert not active
    return done, per_call


def expected_tokens(prompt, n):
    seq, out = list(prompt), []
    for _ in range(n):
        t = FakeModel.next_token(seq)
        out.append(t)
        seq.append(t)
    return out


def test_contract_passes_reference_admission_rules_and_warmup_binds_it():
    be = backend()
    c = be.batch_contract()
    reference_contract_checks(c, "gpt-oss-test", "c1")
    assert c["reserved_state_bytes"] == 4 * 1000 and c["max_context_tokens"] == 64
    w = be.warmup()
    assert w["batch_contract_sha256"] == contract_digest(c) and w["proof_verified"] is True
    assert w["committed_tokens"] == 2
    assert contract_digest(c) == hashlib.sha256(json.dumps(c, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def test_chunked_prefill_then_one_token_per_call():
    be = backend()
    a, b = Job("a", list(range(3, 14)), 5), Job("b", [7, 8], 3)          # 11 tokens = 3 chunks of 4
    done, per_call = run_worker(be, [a, b])
    assert a.tokens == expected_tokens(range(3, 14), 5) and b.tokens == expected_tokens([7, 8], 3)
    assert per_call[0] == {"a": 0, "b": 1} and per_call[1] == {"a": 0, "b": 1} and per_call[2]["a"] == 1
    assert be.model.steps[0] == [4, 2] and be.model.steps[1] == [4, 1]
    for j in (a, b):
        assert done[j.id]["tokens"] == j.checkpoint() and done[j.id]["finish_reason"] == "length"
        assert be.verify_result_proof(j, done[j.id])
    bad = dict(done["a"], tokens=done["a"]["tokens"][:-1] + [0])
    assert not be.verify_result_proof(a, bad)
    assert not be.jobs and sorted(be.free_slots) == [0, 1, 2, 3]


def test_tokens_independent_of_batch_mates_and_join_order():
    solo = backend()
    x = Job("x", [1, 2, 3, 4, 5, 6], 4)
    run_worker(solo, [x])
    mixed = backend()
    y, z = Job("x", [1, 2, 3, 4, 5, 6], 4), Job("z", list(range(20)), 6)
    run_worker(mixed, [z, y])
    assert x.tokens == y.tokens


def test_one_lane_cancel_does_not_stop_the_others():
    be = backend()
    a, b = Job("a", [1, 2, 3], 6), Job("b", [4, 5], 3)
    done, _ = run_worker(be, [a, b], cancel={"a"})
    assert isinstance(done["a"], JobCancelled) and done["b"]["tokens"] == expected_tokens([4, 5], 3)


def test_ring_errors_propagate():
    be = backend()
    j = Job("a", [1, 2], 3)

    def emit(tok):
        raise RingUnavailable("batch ring lease expired")
    with pytest.raises(RingUnavailable):
        be.advance_batch([j], emit={"a": emit}, cancel_check={"a": lambda: None}, max_step_tokens=1)


def test_recovered_job_does_not_reemit_committed_tokens():
    full = expected_tokens([9, 9, 1], 5)
    be = backend()
    j = Job("r", [9, 9, 1], 5, tokens=full[:2])
    run_worker(be, [j])
    assert j.tokens == full


def test_bad_prompt_is_a_job_failure_not_a_ring_failure():
    be = backend()
    long_job, ok = Job("long", list(range(40)), 2), Job("ok", [1], 2)
    done, _ = run_worker(be, [long_job, ok])
    assert isinstance(done["long"], ValueError) and done["ok"]["tokens"] == expected_tokens([1], 2)


def test_eos_stops_a_job():
    first = expected_tokens([3, 1, 4], 1)[0]
    be = backend(eos_ids=[first])
    j = Job("e", [3, 1, 4], 8)
    done, _ = run_worker(be, [j])
    assert done["e"]["finish_reason"] == "stop" and j.tokens == [first]
