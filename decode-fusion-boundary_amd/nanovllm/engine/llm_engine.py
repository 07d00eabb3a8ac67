"""Engine loop (reference ``engine/llm_engine.py:19-218``): schedule -> run -> postprocess."""

from __future__ import annotations

import os
import warnings
from dataclasses import fields
from time import perf_counter

from nanovllm.config import Config
from nanovllm.engine.model_runner import ModelRunner
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.metrics import MetricsCollector
from nanovllm.sampling_params import SamplingParams


class LLMEngine:
    def __init__(self, model, **kwargs):
        names = {f.name for f in fields(Config)}
        config = Config(model, **{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        Sequence.block_size = config.kvcache_block_size
        if config.decode_backend == "megakernel" and config.max_model_len > 2048:
            warnings.warn(
                f"decode_backend={config.decode_backend!r} requires max_model_len <= 2048 "
                f"(got {config.max_model_len}); every request will fall back to the torch path. "
                "Pass max_model_len=2048 to actually use the Megakernel.",
                RuntimeWarning,
            )
        self._exited = False
        self.model_runner = ModelRunner(config, 0, None)
        self.tokenizer = None
        if any(f.startswith("tokenizer") for f in os.listdir(config.model)):
            from transformers import AutoTokenizer

            self.tokenizer = AutoTokenizer.from_pretrained(config.model, use_fast=True)
            config.eos = self.tokenizer.eos_token_id
        else:  # synthetic model directories ship no tokenizer: prompts are token ids
            eos = getattr(config.hf_config, "eos_token_id", -1)
            config.eos = eos if isinstance(eos, int) else -1
        self.scheduler = Scheduler(config)

    def exit(self):
        if self._exited:
            return
        self._exited = True
        try:
            self.model_runner.call("exit")
        except Exception as exc:  # noqa: BLE001
            warnings.warn(f"nano-vLLM cleanup warning: {exc}", RuntimeWarning)

    def add_request(self, prompt, sampling_params: SamplingParams):
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("this model directory has no tokenizer; pass token id lists")
            prompt = self.tokenizer.encode(prompt)
        seq = Sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq

    def step(self, metrics: MetricsCollector | None = None):
        seqs, is_prefill = self.scheduler.schedule()
        num_tokens = sum(s.num_scheduled_tokens for s in seqs) if is_prefill else -len(seqs)
        before = {s.seq_id: len(s.completion_token_ids) for s in seqs}
        t0 = perf_counter()
        token_ids = self.model_runner.call("run", seqs, is_prefill)
        duration = perf_counter() - t0
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        if metrics is not None:
            metrics.record_step(seqs, is_prefill, duration, self.model_runner.last_backend_used,
                                self.model_runner.last_fallback_reason)
            now = perf_counter()
            for s in seqs:
                for _ in range(len(s.completion_token_ids) - before[s.seq_id]):
                    metrics.record_token(s.seq_id, now)
        outputs = [(s.seq_id, s.completion_token_ids) for s in seqs if s.is_finished]
        return outputs, num_tokens

    def is_finished(self):
        return self.scheduler.is_finished()

    def _generate(self, prompts, sampling_params, metrics):
        started = perf_counter()
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        for prompt, sp in zip(prompts, sampling_params):
            seq = self.add_request(prompt, sp)
            if metrics is not None:
                metrics.add_request(seq.seq_id, seq.num_prompt_tokens, perf_counter())
        outputs = {}
        while not self.is_finished():
            out, _ = self.step(metrics)
            for seq_id, token_ids in out:
                outputs[seq_id] = token_ids
        ordered = [outputs[k] for k in sorted(outputs)]
        results = [{"text": self.tokenizer.decode(ids) if self.tokenizer else None, "token_ids": ids}
                   for ids in ordered]
        report = None
        if metrics is not None:
            report = metrics.report(wall_time=perf_counter() - started, scheduler_stats=self.scheduler.stats())
        return results, report

    def generate(self, prompts, sampling_params, use_tqdm: bool = False):
        return self._generate(prompts, sampling_params, None)[0]

    def generate_with_metrics(self, prompts, sampling_params, use_tqdm: bool = False) -> dict:
        collector = MetricsCollector(self.config.decode_backend)
        outputs, report = self._generate(prompts, sampling_params, collector)
        return {"outputs": outputs, "metrics": report}
