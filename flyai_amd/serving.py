"""A qualified continuous-batch backend for the reference's ring scheduler (schema
``shard-token-batch/1``, ``shard/continuous_batch.py:18-48``), serving a GPT-OSS-shaped model on one
MI355X through libflyai_stage.

* ``GptOssModel`` -- embedding gather -> the ragged stage step over every layer -> final RMSNorm ->
  lm_head + greedy pick, all launches of the C ABI (``phase0/specpipe.py:595-616``, ``:779-801``).
  One ``step`` runs every active job at once: prefill chunks and single-token decode rows share one
  flat token batch (``RaggedStage.forward``), and only each job's last row reaches the lm_head (as
  ``specpipe.py:794-795`` does for prefill).
* ``GptOssBatchBackend`` -- ``batch_contract`` / ``advance_batch`` / ``release_batch_job`` with the
  semantics ``ContinuousRingWorker`` and ``RingPool.execute_batch_step`` rely on
  (``shard/continuous_batch.py:98-156``, ``shard/ring_pool.py:627-700``): per-job KV state owned by
  the backend between calls, at most one committed token per job per call, prefill in
  ``prefill_chunk_tokens`` chunks, per-job cancellation, and a result carrying
  ``tokens == job.checkpoint()`` plus a proof that ``verify_result_proof`` re-checks.

Proofs.  The reference's serving rings attach Ed25519 receipt chains (``shard/receipt.py``), which
belong to its auth layer, outside this hot path.  A ``prover`` / ``verifier`` pair plugs them in; the
default ``DigestProver`` binds (job id, committed tokens, contract digest) with SHA-256, and
``verify_result_proof`` recomputes it.
"""
import hashlib
import json

import numpy as np
import torch

from . import _lib, ops
from .runtime import KVWorkspace, RaggedStage

SCHEMA = "shard-token-batch/1"
CONTRACT_KEYS = ("schema", "model_id", "cohort_id", "source_sha256", "runtime_config_sha256",
                 "numerical_contract", "max_jobs", "max_step_tokens", "max_prompt_tokens", "max_new_tokens",
                 "max_context_tokens", "per_job_state_bytes", "reserved_state_bytes", "prefill_chunk_tokens",
                 "cancellation")
NUMERICAL_CONTRACT = ("flyai-amd/gfx950 greedy/1: bf16 activations, MXFP4 experts with fp32 accumulation, "
                      "per-row fixed reduction orders (a job's tokens do not depend on its batch mates), "
                      "bf16 logits, first-maximum argmax")
# the reference's per-job stop signals (shard/service_queue.py JobCancelled / JobExpired) are recorded
# as that job's outcome; any other exception from a callback fails the ring, as it does there
STOP_ERRORS = ("JobCancelled", "JobExpired")


def contract_digest(value):
    """SHA-256 of the canonical JSON of a contract (the digest ``ring.batch_contract_sha256`` holds,
    ``shard/continuous_batch.py:13-15``)."""
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":"),
                                     allow_nan=False).encode()).hexdigest()


def _sha256_file(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for blk in iter(lambda: f.read(1 << 20), b""):
            h.update(blk)
    return h.hexdigest()


class GptOssModel:
    """A whole GPT-OSS-shaped model on one GPU: ``embed`` bf16 [V, H], ``layers`` (LayerWeights),
    ``norm_w`` fp32 [H], ``lm_head`` bf16 [V, H] (re-packed once), KV for ``max_jobs`` sequences of
    ``max_context`` positions."""

    def __init__(self, shape, layers, embed, norm_w, lm_head, rotary, max_jobs, max_context,
                 max_step_rows, device="cuda"):
        self.shape, self.device = shape, torch.device(device)
        self.embed, self.norm_w = embed, norm_w
        self.vocab = int(embed.shape[0])
        if tuple(lm_head.shape) != (self.vocab, shape.hidden) or tuple(embed.shape) != (self.vocab, shape.hidden):
            raise ValueError("embed and lm_head must be [vocab, hidden]")
        self.lm_packed = ops.bf16_tile_repack(lm_head)
        self.max_jobs, self.max_context, self.max_step_rows = max_jobs, max_context, max_step_rows
        self.kv = KVWorkspace(len(layers), max_jobs, max_context, shape.n_kv_heads, shape.head_dim, device)
        self.stage = RaggedStage(shape, layers, rotary, self.kv, max_step_rows, max_jobs, device=device)
        self.n_layers = len(layers)

    @property
    def per_job_state_bytes(self):
        return self.n_layers * 2 * self.kv.slab * 2

    def step(self, chunks, starts, slots, pick):
        """One ragged step.  chunks[i]: token ids fed for sequence i at positions starts[i]...; slots[i]
        its KV slot; pick[i]: whether to return the greedy token after its last row.  Returns a list
        with a token id (or None) per sequence."""
        q_lens = [len(c) for c in chunks]
        T = sum(q_lens)
        if T > self.max_step_rows:
            raise ValueError(f"step of {T} rows exceeds {self.max_step_rows}")
        flat = torch.tensor([t for c in chunks for t in c], dtype=torch.int32).to(self.device, non_blocking=True)
        h = ops.embed_gather(self.embed, flat)
        self.stage.forward(h, q_lens, starts, slots)
        xn = ops.rmsnorm(h, self.norm_w, self.shape.rms_eps)
        ends = np.cumsum(q_lens) - 1
        rows = [int(ends[i]) for i in range(len(chunks)) if pick[i]]
        out = [None] * len(chunks)
        if not rows:
            return out
        toks = []
        for r0 in range(0, len(rows), 64):
            sel = torch.tensor(rows[r0:r0 + 64], dtype=torch.int32).to(self.device, non_blocking=True)
            toks += ops.lm_head_argmax(xn, self.lm_packed, self.vocab, rows=sel).cpu().tolist()
        it = iter(toks)
        for i in range(len(chunks)):
            if pick[i]:
                out[i] = next(it)
        return out


class DigestProver:
    """Default proof: SHA-256 over (job id, committed tokens, contract digest)."""

    scope = "complete_final_attempt"

    def __init__(self, contract_sha256):
        self.contract_sha256 = contract_sha256

    def digest(self, job_id, tokens):
        return hashlib.sha256(json.dumps([str(job_id), [int(t) for t in tokens], self.contract_sha256],
                                         separators=(",", ":")).encode()).hexdigest()

    def prove(self, job, tokens):
        return {"verified": True, "scope": self.scope, "sha256": self.digest(job.id, tokens)}

    def verify(self, job, value):
        proof = value.get("proof", {})
        return (proof.get("verified") is True and proof.get("scope") == self.scope
                and proof.get("sha256") == self.digest(job.id, value.get("tokens", [])))


class _JobState:
    __slots__ = ("slot", "context", "fed", "pending")

    def __init__(self, slot, context):
        self.slot, self.context, self.fed, self.pending = slot, context, 0, None


class GptOssBatchBackend:
    """The ``shard-token-batch/1`` backend trio over ``GptOssModel``.

    tokenize(payload) -> prompt token ids (the reference tokenizes before the ring; it is not part of
    this path).  A job that a ring recovered with committed tokens re-prefills prompt + those tokens
    and continues without re-emitting them (``continuous_batch.py:120-124``)."""

    def __init__(self, model: GptOssModel, *, model_id, cohort_id, tokenize, max_prompt_tokens,
                 max_new_tokens, prefill_chunk_tokens, max_step_tokens=1, eos_ids=(), source_sha256=None,
                 prover=None):
        if not 1 <= model.max_jobs <= 32:
            raise ValueError("max_jobs must be in [1, 32] (scheduler limit)")
        if not 1 <= max_step_tokens <= 64:
            raise ValueError("max_step_tokens must be in [1, 64]")
        if not 1 <= prefill_chunk_tokens <= max_prompt_tokens:
            raise ValueError("prefill_chunk_tokens must be in [1, max_prompt_tokens]")
        if max_prompt_tokens >= model.max_context or max_new_tokens > model.max_context:
            raise ValueError("token bounds exceed the context capacity")
        if model.max_jobs * prefill_chunk_tokens > model.max_step_rows:
            raise ValueError("max_step_rows must hold a prefill chunk for every job")
        self.model, self.model_id, self.cohort_id = model, model_id, cohort_id
        self.tokenize = tokenize
        self.max_prompt_tokens, self.max_new_tokens = max_prompt_tokens, max_new_tokens
        self.prefill_chunk_tokens, self.max_step_tokens = prefill_chunk_tokens, max_step_tokens
        self.eos_ids = frozenset(int(t) for t in eos_ids)
        self.source_sha256 = source_sha256 or _sha256_file(_lib.LIB_PATH)
        self._contract = self._make_contract()
        self.prover = prover or DigestProver(contract_digest(self._contract))
        self.jobs = {}
        self.free_slots = list(range(model.max_jobs - 1, -1, -1))

    # ---- contract -------------------------------------------------------------------------------
    def _make_contract(self):
        m, sh = self.model, self.model.shape
        runtime = {"abi": int(_lib.lib().flyai_abi_version()), "layers": m.n_layers, "hidden": sh.hidden,
                   "experts": sh.n_experts, "top_k": sh.top_k, "vocab": m.vocab, "max_jobs": m.max_jobs,
                   "max_context": m.max_context, "max_step_rows": m.max_step_rows,
                   "prefill_chunk": self.prefill_chunk_tokens, "eos": sorted(self.eos_ids)}
        per_job = m.per_job_state_bytes
        return {"schema": SCHEMA, "model_id": self.model_id, "cohort_id": self.cohort_id,
                "source_sha256": self.source_sha256,
                "runtime_config_sha256": hashlib.sha256(json.dumps(runtime, sort_keys=True).encode()).hexdigest(),
                "numerical_contract": NUMERICAL_CONTRACT, "max_jobs": m.max_jobs,
                "max_step_tokens": self.max_step_tokens, "max_prompt_tokens": self.max_prompt_tokens,
                "max_new_tokens": self.max_new_tokens, "max_context_tokens": m.max_context,
                "per_job_state_bytes": per_job, "reserved_state_bytes": per_job * m.max_jobs,
                "prefill_chunk_tokens": self.prefill_chunk_tokens, "cancellation": "per_job"}

    def batch_contract(self):
        return dict(self._contract)

    def ready(self):
        return True, "ready"

    def warmup(self, timeout_s=300.0):
        """Generate twice from a fixed prompt in a free slot; the warmup is verified when both runs
        commit the same tokens (the step is deterministic).  Binds the contract digest."""
        if self.jobs:
            raise RuntimeError("warmup requires an idle backend")
        prompt = [i % self.model.vocab for i in (1, 2, 3, 5, 8)]
        runs = []
        for _ in range(2):
            slot = self.free_slots[-1]
            toks = []
            t = self.model.step([prompt], [0], [slot], [True])[0]
            toks.append(t)
            t = self.model.step([[t]], [len(prompt)], [slot], [True])[0]
            toks.append(t)
            runs.append(toks)
        return {"proof_verified": runs[0] == runs[1], "committed_tokens": len(runs[0]), "tokens": runs[0],
                "batch_contract_sha256": contract_digest(self.batch_contract())}

    # ---- jobs -----------------------------------------------------------------------------------
    def _admit(self, job):
        prompt = [int(t) for t in self.tokenize(job.payload)]
        committed = [int(t) for t in job.tokens]
        if not 1 <= len(prompt) <= self.max_prompt_tokens:
            raise ValueError(f"prompt of {len(prompt)} tokens outside [1, {self.max_prompt_tokens}]")
        if job.max_new > self.max_new_tokens or len(prompt) + job.max_new > self.model.max_context:
            raise ValueError("job exceeds the contract's token bounds")
        if any(not 0 <= t < self.model.vocab for t in prompt + committed):
            raise ValueError("token id outside the vocabulary")
        if not self.free_slots:
            raise RuntimeError("no free KV slot (more live jobs than max_jobs)")
        st = _JobState(self.free_slots.pop(), prompt + committed)
        self.jobs[job.id] = st
        return st

    def _result(self, job, reason):
        tokens = job.checkpoint()
        return {"tokens": tokens, "finish_reason": reason, "proof": self.prover.prove(job, tokens)}

    def advance_batch(self, jobs, *, emit, cancel_check, max_step_tokens):
        """One ragged step over every job: a prefill chunk for jobs still prefilling, one decode row
        for the others; each job whose step ends its context commits one greedy token.  Returns
        {job.id: None | Exception | result} for every job."""
        if not 1 <= max_step_tokens <= self.max_step_tokens:
            raise ValueError("max_step_tokens outside the contract")
        out = {}
        live = []
        for job in jobs:
            try:
                cancel_check[job.id]()
                st = self.jobs.get(job.id) or self._admit(job)
                if len(job.tokens) >= job.max_new:
                    out[job.id] = self._result(job, "length")
                    continue
                live.append((job, st))
            except Exception as error:  # noqa: BLE001 -- classified below
                if type(error).__name__ in STOP_ERRORS or isinstance(error, ValueError):
                    out[job.id] = error
                else:
                    raise
        if live:
            chunks, starts, slots, pick = [], [], [], []
            for job, st in live:
                if st.fed < len(st.context):
                    c = st.context[st.fed:st.fed + self.prefill_chunk_tokens]
                    pick.append(st.fed + len(c) == len(st.context))
                else:
                    c = [st.pending]
                    pick.append(True)
                chunks.append(c)
                starts.append(st.fed)
                slots.append(st.slot)
            toks = self.model.step(chunks, starts, slots, pick)
            for (job, st), c, tok in zip(live, chunks, toks):
                st.fed += len(c)
                if tok is None:
                    out[job.id] = None
                    continue
                st.pending = tok
                try:
                    emit[job.id](tok)
                except Exception as error:  # noqa: BLE001
                    if type(error).__name__ in STOP_ERRORS:
                        out[job.id] = error
                        continue
                    raise
                if tok in self.eos_ids:
                    out[job.id] = self._result(job, "stop")
                elif len(job.tokens) >= job.max_new:
                    out[job.id] = self._result(job, "length")
                else:
                    out[job.id] = None
        for job in jobs:
            out.setdefault(job.id, None)
        return out

    def verify_result_proof(self, job, value):
        return self.prover.verify(job, value)

    def release_batch_job(self, job_id):
        st = self.jobs.pop(job_id, None)
        if st is not None:
            self.free_slots.append(st.slot)
