"""The single-request engine the reference's server drives (src/mlx_dspark/server.py:75-370),
wired to this package: no HTTP here, only what the request handlers call.

``Engine`` holds the loaded target / drafter and turns prompt ids into a GenResult:
mode dispatch (dspark, dflash, lookup, baseline greedy), prefix KV reuse across requests for
the modes whose generate functions take caches back (dspark, lookup, baseline; DFlash starts
fresh, as in the reference), and the throughput stats behind ``metrics()``. Every request runs
on one worker thread, one at a time, so caches and device work stay on a single thread.
"""

from __future__ import annotations

import time
from concurrent.futures import ThreadPoolExecutor

from .generate import GenResult, dflash_generate, greedy_generate, speculative_generate
from .lookup import lookup_generate
from .prefix_cache import PrefixCache, target_cache_reusable

MODES = ("dspark", "dflash", "lookup", "baseline")


class Engine:
    """``target`` (Target), ``tokenizer``, ``drafter`` (DSpark / DFlash drafter or None);
    ``max_ctx`` sizes the reusable caches (requests that would outgrow it run on fresh caches
    sized by the generate functions)."""

    def __init__(self, target, tokenizer, drafter, *, mode: str, model_id: str, target_repo: str = "",
                 drafter_repo: str | None = None, max_draft_tokens: int | None = None,
                 confidence_threshold: float = 0.0, template_defaults: dict | None = None,
                 prefix_cache: bool = True, prefix_cache_dir: str | None = None, prefix_cache_max_ram_mb: int = 0,
                 cap_controller=None, sampling_defaults: dict | None = None, default_max_tokens: int = 2048,
                 max_tokens_cap: int = 32768, prefix_cache_slots: int = 2, lookup_drafts: bool = True,
                 executor: ThreadPoolExecutor | None = None, max_ctx: int = 16384):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        if mode in ("dspark", "dflash") and drafter is None:
            raise ValueError(f"mode {mode!r} needs a drafter")
        self.target, self.tokenizer, self.drafter = target, tokenizer, drafter
        self.mode, self.model_id = mode, model_id
        self.target_repo, self.drafter_repo = target_repo, drafter_repo
        self.max_draft_tokens = max_draft_tokens
        self.confidence_threshold = confidence_threshold
        self.cap_controller = cap_controller
        self.sampling_defaults = dict(sampling_defaults or {})
        self.template_defaults = dict(template_defaults or {})
        self.default_max_tokens, self.max_tokens_cap = default_max_tokens, max_tokens_cap
        self.prefix_cache_slots = max(1, prefix_cache_slots)
        self.lookup_drafts = lookup_drafts
        self.max_ctx = int(max_ctx)
        self.prefix = self._build_prefix_cache(prefix_cache, prefix_cache_dir, prefix_cache_max_ram_mb)
        self._executor = executor or ThreadPoolExecutor(max_workers=1, thread_name_prefix="dsk-gen")
        self.created = int(time.time())
        self.stats = {"requests": 0, "prompt_tokens": 0, "completion_tokens": 0, "generation_seconds": 0.0,
                      "sum_accept_len": 0.0}

    def _build_prefix_cache(self, enabled, l2_dir, max_ram_mb):
        if not enabled or self.mode == "dflash":
            return None
        make_cache = lambda: self.target.make_cache(max_ctx=self.max_ctx)  # noqa: E731
        if not target_cache_reusable(make_cache()):
            return None
        make_ctx = (lambda: self.drafter.make_ctx_cache(max_ctx=self.max_ctx)) if self.mode == "dspark" else None
        return PrefixCache(make_cache, make_ctx, l2_dir=l2_dir, max_ram_bytes=max(0, max_ram_mb) * 1024 * 1024,
                           slots=self.prefix_cache_slots)

    @classmethod
    def load(cls, *, mode: str = "dspark", model: str | None = None, drafter: str | None = None,
             drafter_bits: int = 4, max_draft_tokens: int | None = None, kv_bits: int | None = None,
             **kw) -> "Engine":
        """Load target (+ drafter) by name (synthetic/* or a local checkpoint directory) and
        build the engine on its own generation thread (server.py:162-250). A learned cap
        controller is not built: pass ``cap_controller=`` to drive the cap."""
        from .load import load_dflash, load_drafter, load_target, resolve_mode

        if max_draft_tokens == "auto":
            raise ValueError("max_draft_tokens='auto' needs a calibrated cap controller (pass cap_controller=)")
        mode, target_repo, drafter_repo = resolve_mode(model, mode=mode, drafter=drafter)
        executor = ThreadPoolExecutor(max_workers=1, thread_name_prefix="dsk-gen")

        def _load():
            tgt, tok = load_target(target_repo, require_tap=mode in ("dspark", "dflash"), kv_bits=kv_bits)
            d = None
            if mode == "dspark":
                d, _ = load_drafter(drafter_repo, bits=drafter_bits, target_args=tgt.model.args)
            elif mode == "dflash":
                d, _ = load_dflash(drafter_repo, bits=drafter_bits, target_args=tgt.model.args)
                d.bind(tgt.model)
            return tgt, tok, d

        tgt, tok, d = executor.submit(_load).result()
        if max_draft_tokens is None and kw.get("cap_controller") is None:
            max_draft_tokens = {"dspark": 2, "lookup": 6}.get(mode)
        model_id = target_repo.rstrip("/").split("/")[-1]
        return cls(tgt, tok, d, mode=mode, model_id=model_id, target_repo=target_repo, drafter_repo=drafter_repo,
                   max_draft_tokens=max_draft_tokens, executor=executor, **kw)

    def close(self) -> None:
        self._executor.shutdown(wait=True)

    # ---- requests
    def generate(self, prompt_ids, *, max_tokens: int, temperature: float, top_p: float = 1.0, top_k: int = 0,
                 presence_penalty: float = 0.0, frequency_penalty: float = 0.0, logprobs: int | None = None,
                 stop=None, seed=None, on_text=None) -> GenResult:
        return self._executor.submit(self._generate_impl, list(prompt_ids), max_tokens, temperature, top_p, top_k,
                                     stop, seed, on_text, presence_penalty, frequency_penalty, logprobs).result()

    def _generate_impl(self, prompt_ids, max_tokens, temperature, top_p, top_k, stop, seed, on_text,
                       presence_penalty=0.0, frequency_penalty=0.0, logprobs=None) -> GenResult:
        cache = ctx = None
        reuse_len = 0
        # a reusable cache has a fixed size: longer requests run on fresh, request-sized caches
        fits = len(prompt_ids) + max_tokens + 64 <= self.max_ctx
        if self.prefix is not None and fits:
            cache, ctx, reuse_len = self.prefix.acquire(prompt_ids)
        try:
            common = dict(prompt_ids=prompt_ids, max_new_tokens=max_tokens, temperature=temperature, top_p=top_p,
                          top_k=top_k, seed=seed, stop=stop, on_text=on_text)
            if self.mode == "dspark":
                res = speculative_generate(self.target, self.tokenizer, self.drafter, cache=cache, ctx_caches=ctx,
                                           reuse_len=reuse_len, max_draft_tokens=self.max_draft_tokens,
                                           cap_controller=self.cap_controller, lookup_drafts=self.lookup_drafts,
                                           confidence_threshold=self.confidence_threshold,
                                           presence_penalty=presence_penalty, frequency_penalty=frequency_penalty,
                                           logprobs=logprobs, **common)
            elif self.mode == "dflash":
                res = dflash_generate(self.target, self.tokenizer, self.drafter, max_draft_tokens=self.max_draft_tokens,
                                      cap_controller=self.cap_controller, **common)
            elif self.mode == "lookup":
                res = lookup_generate(self.target, self.tokenizer, cache=cache, reuse_len=reuse_len,
                                      max_draft_tokens=self.max_draft_tokens or 6, **common)
            else:
                res = greedy_generate(self.target, self.tokenizer, cache=cache, reuse_len=reuse_len,
                                      presence_penalty=presence_penalty, frequency_penalty=frequency_penalty,
                                      logprobs=logprobs, **common)
        except BaseException:
            if self.prefix is not None:          # never keep a cache that may be out of step
                self.prefix.reset()
            raise
        if self.prefix is not None and cache is not None:
            self.prefix.store(cache, ctx, prompt_ids, res.token_ids)
        s = self.stats
        s["requests"] += 1
        s["prompt_tokens"] += len(prompt_ids)
        s["completion_tokens"] += res.num_tokens
        s["generation_seconds"] += res.seconds
        s["sum_accept_len"] += res.mean_accept_len * res.num_tokens
        return res

    def spec_info(self, res: GenResult) -> dict:
        info = {"mode": self.mode, "accept_len": round(res.mean_accept_len, 3),
                "tokens_per_sec": round(res.tokens_per_sec, 1), "target_forwards": res.target_forwards}
        if self.cap_controller is not None:
            info["cap"] = self.cap_controller.cap
        if res.lookup_rounds:
            info["lookup_rounds"] = res.lookup_rounds
        return info

    def metrics(self) -> dict:
        s = self.stats
        ct = s["completion_tokens"]
        ctrl = self.cap_controller
        return {"model": self.model_id, "mode": self.mode, "requests": s["requests"],
                "prompt_tokens": s["prompt_tokens"], "completion_tokens": ct,
                "mean_accept_len": round(s["sum_accept_len"] / ct, 3) if ct else 0.0,
                "mean_tokens_per_sec": round(ct / s["generation_seconds"], 1) if s["generation_seconds"] else 0.0,
                "prefix_cache": self.prefix.info() if self.prefix is not None else {"enabled": False},
                "auto_cap": ctrl.info() if ctrl is not None and hasattr(ctrl, "info") else None}
