"""Deterministic stand-ins for the continuous-batching executors, used to record and replay the
scheduler's event sequence. They change request state exactly as run_prefill_chunk /
run_decode_step do (src/serving/continuous_generate.py:82-276 of the reference) but take a
runtime computed from the batch shape instead of timing a model, and pick token ids by formula.
Imports nothing from either implementation, so both can drive their scheduler with it."""


def make_executors(vocab: int = 5000):
    def prefill(batch, chunk_size, now, event_id):
        chunk_start = batch[0].prompt_tokens_processed
        lens = [max(min(chunk_size, r.prompt_len - chunk_start), 0) for r in batch]
        runtime = 0.25 + 0.002 * sum(lens) + 0.05 * len(batch)
        finish = now + runtime
        done, first = [], 0
        for i, r in enumerate(batch):
            if r.start_time_ms is None:
                r.start_time_ms = now
                r.batch_id = event_id
            r.scheduler_mode = "continuous"
            r.prompt_tokens_processed = chunk_start + lens[i]
            if r.prompt_tokens_processed >= r.prompt_len:
                r.generated_token_ids.append((r.request_id * 7 + 1) % vocab)
                first += 1
                if r.first_token_time_ms is None:
                    r.first_token_time_ms = finish
                if r.num_generated_tokens >= r.max_new_tokens:
                    r.phase = "finished"
                    r.finish_time_ms = finish
                    done.append(r)
                else:
                    r.phase = "decode"
            else:
                r.phase = "prefill"
        return {
            "batch_runtime_ms": runtime, "requests_completed": done, "batch_size": len(batch),
            "tokens_scheduled": sum(lens), "phase": "prefill",
            "prompt_len": max(r.prompt_len for r in batch), "max_new_tokens": max(r.max_new_tokens for r in batch),
            "prefill_tokens": sum(lens), "decode_tokens": first, "decode_kernel_tokens": 0,
            "prefill_runtime_ms": runtime, "decode_runtime_ms": 0.0, "decode_ms_per_token": 0.0,
            "padding_waste_tokens": len(batch) * max(lens) - sum(lens),
        }

    def decode(batch, now, event_id):
        runtime = 0.3 + 0.04 * len(batch)
        finish = now + runtime
        done = []
        for r in batch:
            if r.start_time_ms is None:
                r.start_time_ms = now
                r.batch_id = event_id
            r.scheduler_mode = "continuous"
            r.generated_token_ids.append((r.request_id * 13 + r.num_generated_tokens) % vocab)
            if r.num_generated_tokens >= r.max_new_tokens:
                r.phase = "finished"
                r.finish_time_ms = finish
                done.append(r)
            else:
                r.phase = "decode"
        return {
            "batch_runtime_ms": runtime, "requests_completed": done, "batch_size": len(batch),
            "tokens_scheduled": len(batch), "phase": "decode",
            "prompt_len": max(r.prompt_len for r in batch), "max_new_tokens": max(r.max_new_tokens for r in batch),
            "prefill_tokens": 0, "decode_tokens": len(batch), "decode_kernel_tokens": len(batch),
            "prefill_runtime_ms": 0.0, "decode_runtime_ms": runtime, "decode_ms_per_token": runtime / len(batch),
        }

    return prefill, decode


EVENT_FIELDS = ("batch_id", "dispatch_time_ms", "finish_time_ms", "batch_size", "batch_runtime_ms", "phase",
                "tokens_scheduled", "prompt_len", "max_new_tokens", "prefill_tokens", "decode_tokens")
REQUEST_FIELDS = ("request_id", "arrival_time_ms", "start_time_ms", "first_token_time_ms", "finish_time_ms",
                  "batch_id", "prompt_len", "max_new_tokens")
