"""GPU: the reference's own callers, replayed against this package from recorded call sites.

tests/golden/call_sites.json (written by tests/golden/extract_call_sites.py, which parses the
reference's src/mlx_dspark/server.py and cli.py with ``ast``) holds, per caller function, the
statements that touch this API in line order: calls (callee, positional and keyword arguments,
where the result goes), plain bindings, the conditions that reach each one, and whether it sits
in a try body or an except handler. ``replay`` below interprets those records: it evaluates the
recorded expressions in an environment standing for the caller's state (the engine's mode and
configuration, a request's parameters, the CLI's arguments), runs the reachable records in
order and, when a call in a try body raises, runs that handler's records and re-raises where
the handler does. Replayed:
  - Engine._build_prefix_cache and Engine._generate_impl (server.py:143-158, :272-329), entered
    through BatchEngine._run_serial's mapping of a request onto _generate_impl's parameters
    (:565-575): two requests per mode, the second reusing the first's KV where the mode allows
    it, and a generation whose on_text raises (the prefix store is reset and the error passes);
  - the continuous-batching session's SpecSlots construction and admissions (BatchEngine.
    _run_session / _admit, :494-563) under a scheduler of this test's own: arrivals are admitted
    as rows retire, and every result is delivered when its row does;
  - BatchEngine._run_batched's batch_generate_baseline call (:577-609);
  - the CLI's generate command in each mode (cli.py:101-167): a positional prompt string, the
    chat template applied unless --no-chat-template, text streamed through on_text, and the
    --max-draft auto path, whose cap controller comes from calibrate (a cost-model tuner this
    package leaves out: a stand-in with a fixed cap takes its place);
  - the CLI's benchmark command (cli.py:328-385): the baseline, lookup and each drafter mode
    at a numeric and the auto cap, over a prompt string.
Token streams are checked against the oracle's greedy decoding (tests/_parity.py); prompts
given as strings are encoded for that check by this test's own tokenizer calls."""

import json
import types
from pathlib import Path

import numpy as np
import pytest

from _parity import check_greedy_stream

pytestmark = pytest.mark.gpu
MIN_MATCH = 8
FIX = json.loads((Path(__file__).parent / "golden" / "call_sites.json").read_text())
FUNCS = {f["function"]: f for f in FIX["functions"]}


# ------------------------------------------------------------------ the driver
class Unbound(Exception):
    """A recorded expression names something the replay's environment does not hold."""


def _lookup(env, name):
    if name in env:
        return env[name]
    if name in BUILTINS:
        return BUILTINS[name]
    parts = name.split(".")
    for i in range(len(parts) - 1, 0, -1):
        head = ".".join(parts[:i])
        if head in env:
            obj = env[head]
            for p in parts[i:]:
                if not hasattr(obj, p):
                    raise Unbound(name)
                obj = getattr(obj, p)
            return obj
    raise Unbound(name)


def _api():
    from mlx_dspark import batch_engine, generate, load, lookup, prefix_cache
    return {"speculative_generate": generate.speculative_generate, "dflash_generate": generate.dflash_generate,
            "greedy_generate": generate.greedy_generate, "lookup_generate": lookup.lookup_generate,
            "SpecSlots": batch_engine.SpecSlots, "batch_generate_baseline": batch_engine.batch_generate_baseline,
            "PrefixCache": prefix_cache.PrefixCache, "target_cache_reusable": prefix_cache.target_cache_reusable,
            "load_target": load.load_target, "load_drafter": load.load_drafter, "load_dflash": load.load_dflash}


BUILTINS = {"max": max, "min": min, "int": int, "len": len, "bool": bool, "str": str, "isinstance": isinstance}
CMP = {"==": lambda a, b: a == b, "!=": lambda a, b: a != b, "is": lambda a, b: a is b,
       "is not": lambda a, b: a is not b, "<": lambda a, b: a < b, "<=": lambda a, b: a <= b,
       ">": lambda a, b: a > b, ">=": lambda a, b: a >= b, "in": lambda a, b: a in b,
       "not in": lambda a, b: a not in b}
BIN = {"+": lambda a, b: a + b, "-": lambda a, b: a - b, "*": lambda a, b: a * b, "//": lambda a, b: a // b,
       "/": lambda a, b: a / b, "%": lambda a, b: a % b}


def _callable(name, env):
    if name in env:
        return env[name]
    if name in BUILTINS:
        return BUILTINS[name]
    api = _api()
    if name in api:
        return api[name]
    return _lookup(env, name)


def ev(x, env):
    """Evaluate one recorded expression (the grammar of tests/golden/extract_call_sites.py)."""
    kind = next(iter(x))
    v = x[kind]
    if kind == "name" or kind == "attr":
        return _lookup(env, v)
    if kind == "const":
        return v
    if kind == "or":
        r = None
        for e in v:
            r = ev(e, env)
            if r:
                return r
        return r
    if kind == "and":
        r = None
        for e in v:
            r = ev(e, env)
            if not r:
                return r
        return r
    if kind == "not":
        return not ev(v, env)
    if kind == "neg":
        return -ev(v, env)
    if kind == "if":
        return ev(v[1], env) if ev(v[0], env) else ev(v[2], env)
    if kind == "cmp":
        return CMP[v[1]](ev(v[0], env), ev(v[2], env))
    if kind == "bin":
        return BIN[v[1]](ev(v[0], env), ev(v[2], env))
    if kind == "item":
        return ev(v[0], env)[ev(v[1], env)]
    if kind == "tuple":
        return tuple(ev(e, env) for e in v)
    if kind == "getattr":
        return getattr(ev(v[0], env), v[1])
    if kind == "call":
        fn = _callable(v, env)
        return fn(*[ev(a, env) for a in x["args"]], **{k: ev(a, env) for k, a in x["kwargs"].items()})
    if kind == "lambda":
        return lambda *a: ev(x["body"], {**env, **dict(zip(v, a))})
    if kind == "fstr":
        return "".join(p if isinstance(p, str) else str(ev(p["expr"], env)) for p in v)
    raise Unbound(kind)


def _reachable(rec, env):
    for c in rec["conditions"]:
        if next(iter(c)) in ("for", "while"):
            continue                            # the test drives loops itself
        try:
            if not ev(c, env):
                return False
        except Unbound:
            return False
    return True


def _assign(env, names, value):
    if len(names) > 1:
        value = list(value)
    for i, n in enumerate(names):
        v = value[i] if len(names) > 1 else value
        if n is None or n == "_":
            continue
        if "." in n:                            # attribute target: set it on the object
            head, attr = n.rsplit(".", 1)
            setattr(_lookup(env, head), attr, v)
        else:
            env[n] = v


def replay(fname, env, provided=(), select=None):
    """Run the recorded statements of ``fname`` in line order against ``env`` (updated in place).
    Names in ``provided`` are the test's own: bindings and calls that would set them are
    skipped. ``select`` filters the records. Returns (calls made, the returned value)."""
    made, ret, failure, handled = [], None, None, False
    for rec in FUNCS[fname]["records"]:
        if select is not None and not select(rec):
            continue
        place = rec["placement"]
        if place == "except":
            if failure is None:
                continue
            handled = True
            if rec.get("handler_as"):
                env[rec["handler_as"]] = failure
        elif place == "try":
            if failure is not None:
                continue
        elif failure is not None:
            if not handled:
                raise failure                   # no handler ran: the exception leaves the function
            failure = None                      # the handler ended without re-raising
        if not _reachable(rec, env):
            continue
        if rec["kind"] == "reraise":
            raise failure
        if rec["kind"] == "bind":
            if any(n in provided for n in rec["names"]):
                continue
            try:
                value = ev(rec["value"], env)
            except Exception:                   # a caller-side value this replay does not model
                continue
            for group in rec["groups"]:
                _assign(env, group, value)
            continue
        names = rec["assign"] or []
        if names and all(n in provided or n == "_" for n in names):
            continue
        fn = _callable(rec["callee"], env)
        args = [ev(a, env) for a in rec["args"]]
        kwargs = {k: ev(a, env) for k, a in rec["kwargs"].items()}
        try:
            res = fn(*args, **kwargs)
        except BaseException as e:
            if place != "try":
                raise
            failure, handled = e, False
            continue
        made.append((rec, res))
        if names == ["return"]:
            ret = res
        elif names:
            _assign(env, names, res)
    if failure is not None and not handled:
        raise failure
    return made, ret


# ------------------------------------------------------------------ models and caller state
@pytest.fixture(scope="module")
def models(dev):
    from mlx_dspark.load import load_dflash_pair, load_pair
    target, tok, d, _ = load_pair("synthetic/tiny", keep_mlx=True)
    t2, tok2, dfl, _ = load_dflash_pair("synthetic/tiny", keep_mlx=True)
    return {"dspark": (target, tok, d), "dflash": (t2, tok2, dfl)}


def _engine(mode, models, max_draft_tokens=None, cap_controller=None):
    """The server Engine's state the recorded statements read (attributes of ``self``)."""
    target, tok, d = models["dflash" if mode == "dflash" else "dspark"]
    return {"self.mode": mode, "self.target": target, "self.tokenizer": tok,
            "self.drafter": d if mode in ("dspark", "dflash") else None, "self.max_draft_tokens": max_draft_tokens,
            "self.cap_controller": cap_controller, "self.lookup_drafts": True, "self.confidence_threshold": 0.0,
            "self.prefix_cache_slots": 2}


def _server(mode, models, **kw):
    """Engine state plus its prefix store, built by the recorded _build_prefix_cache."""
    env = _engine(mode, models, **kw)
    _, prefix = replay("Engine._build_prefix_cache", {**env, "enabled": True, "l2_dir": None, "max_ram_mb": 0})
    env["self.prefix"] = prefix
    return env


def _request(env, prompt_ids, max_tokens, on_text=None, **params):
    """A request through BatchEngine._run_serial into Engine._generate_impl: the recorded call
    maps the job's parameters onto _generate_impl's parameters."""
    gen_params = FUNCS["Engine._generate_impl"]["params"][1:]

    def generate_impl(*args):
        local = {**env, **dict(zip(gen_params, args))}
        made, _ = replay("Engine._generate_impl", local)
        assert sum(r["callee"].endswith("_generate") for r, _ in made) == 1, "one generate call per request"
        return local["res"]

    p = {"max_tokens": max_tokens, "temperature": 0.0, "top_p": 1.0, "top_k": 0, "stop": None, "seed": None,
         "presence_penalty": 0.0, "frequency_penalty": 0.0, "logprobs": None, **params}
    job = types.SimpleNamespace(prompt_ids=prompt_ids, params=p, on_text=on_text, result=None, error=None)
    replay("BatchEngine._run_serial", {"self.engine._generate_impl": generate_impl, "job": job})
    if job.error is not None:
        raise job.error
    return job.result


# ------------------------------------------------------------------ server
@pytest.mark.parametrize("mode", ["dspark", "baseline", "lookup", "dflash"])
def test_server_single_request_sequence(dev, models, mode):
    print(f"server sequence mode={mode}", flush=True)
    mdt = {"dspark": 2, "lookup": 6}.get(mode)
    env = _server(mode, models, max_draft_tokens=mdt)
    target = env["self.target"]
    V = target.model.args.vocab_size
    rng = np.random.default_rng(31)
    t1 = rng.integers(0, V, 48).tolist()
    r1 = _request(env, t1, 16)
    t2 = t1 + r1.token_ids + rng.integers(0, V, 10).tolist()
    r2 = _request(env, t2, 16)
    for prompt, res in ((t1, r1), (t2, r2)):
        assert 16 <= res.num_tokens <= 16 + (mdt or 0)     # lookup commits whole rounds
        check_greedy_stream(target.model, prompt, res.token_ids, MIN_MATCH)
    prefix = env["self.prefix"]
    if mode == "dflash":
        assert prefix is None                               # no prefix store for DFlash
    else:
        info = prefix.info()
        assert info["hits"] == 1 and info["reused_tokens"] == len(t1) + len(r1.token_ids) - 1
        assert len(info["slots"]) == 1 and info["slots"][0]["tokens"] == len(t2) + 15


def test_server_resets_the_prefix_store_when_a_generation_raises(dev, models):
    env = _server("dspark", models, max_draft_tokens=2)
    V = env["self.target"].model.args.vocab_size
    t1 = np.random.default_rng(5).integers(0, V, 40).tolist()
    _request(env, t1, 8)
    assert len(env["self.prefix"].info()["slots"]) == 1

    def boom(text):
        raise KeyboardInterrupt

    with pytest.raises(KeyboardInterrupt):
        _request(env, t1 + [1, 2], 8, on_text=boom)
    assert env["self.prefix"].info()["slots"] == []
    res = _request(env, t1, 8)
    check_greedy_stream(env["self.target"].model, t1, res.token_ids, MIN_MATCH)


def test_server_batching_session_sequence(dev, models):
    target, tok, d = models["dspark"]
    V = target.model.args.vocab_size
    rng = np.random.default_rng(41)
    jobs = [types.SimpleNamespace(id=i, prompt_ids=rng.integers(0, V, int(n)).tolist(), on_text=None, error=None,
                                  params={"max_tokens": int(m), "stop": None})
            for i, (n, m) in enumerate([(40, 10), (70, 24), (33, 6), (52, 16), (45, 12), (61, 8)])]
    eng = types.SimpleNamespace(target=target, tokenizer=tok, drafter=d, max_draft_tokens=None, cap_controller=None)
    env = {"self.engine": eng, "self.max_batch": 3, "jobs": jobs[:3], "eng": eng}
    made, _ = replay("BatchEngine._run_session", env, provided={"eng"},
                     select=lambda r: r["kind"] == "call" and r["callee"] == "SpecSlots")
    slots = env["slots"]

    def admit(job):
        replay("BatchEngine._admit", {"slots": slots, "job": job})
        assert job.error is None

    waiting, arrivals = list(jobs[:3]), list(jobs[3:])     # the rest arrive while the session runs
    done, order, peak, steps = {}, [], 0, 0
    while slots.n_active or waiting or arrivals:
        if steps % 2 == 1 and arrivals:
            waiting.append(arrivals.pop(0))
        while waiting and slots.has_free_slot:
            admit(waiting.pop(0))
        peak = max(peak, slots.n_active)
        for job, res in slots.step():
            done[job.id] = res
            order.append((job.id, steps))
        steps += 1
    assert sorted(done) == list(range(len(jobs))) and peak == 3
    assert order[0][1] < order[-1][1]                     # rows retire as they finish
    for job in jobs:
        res = done[job.id]
        mt = job.params["max_tokens"]
        # a round commits up to cap + 1 tokens, so a row may end past its limit (as in the reference)
        assert mt <= res.num_tokens <= mt + 2
        check_greedy_stream(target.model, job.prompt_ids, res.token_ids, min(MIN_MATCH, mt))


def test_server_batched_baseline(dev, models):
    target, tok, _ = models["dspark"]
    V = target.model.args.vocab_size
    rng = np.random.default_rng(43)
    jobs = [types.SimpleNamespace(prompt_ids=rng.integers(0, V, int(n)).tolist(), on_text=None, result=None,
                                  error=None, params={"max_tokens": int(m), "stop": None})
            for n, m in [(30, 12), (55, 7), (41, 10)]]
    env = {"self.engine": types.SimpleNamespace(target=target, tokenizer=tok), "jobs": jobs, "key": (0.0, 1.0, 0),
           "prompts": [j.prompt_ids for j in jobs], "max_toks": [j.params["max_tokens"] for j in jobs],
           "on_texts": [j.on_text for j in jobs], "stops": [j.params["stop"] for j in jobs]}
    made, _ = replay("BatchEngine._run_batched", env, provided={"prompts", "max_toks", "on_texts", "stops"},
                     select=lambda r: r["kind"] != "bind" or r["names"] == ["temp", "top_p", "top_k"])
    assert [r["callee"] for r, _ in made] == ["batch_generate_baseline"]
    for j, res in zip(jobs, env["res"]):
        assert res.num_tokens == j.params["max_tokens"]
        check_greedy_stream(target.model, j.prompt_ids, res.token_ids, min(MIN_MATCH, j.params["max_tokens"]))


# ------------------------------------------------------------------ CLI
class ChatTokenizer:
    """The synthetic tokenizer with a chat template: a user turn is framed by fixed marker ids,
    so a prompt encoded with the template differs from the plain encoding."""

    chat_template = "user-turn"

    def __init__(self, base):
        self.base = base
        self.vocab_size, self.eos_token_id, self.unk_token_id = base.vocab_size, None, None

    def encode(self, text):
        return self.base.encode(text)

    def decode(self, ids):
        return self.base.decode(ids)

    def apply_chat_template(self, messages, add_generation_prompt=True, **_):
        ids = []
        for m in messages:
            ids += [3, 5] + self.encode(m["content"]) + [7]
        return ids + ([3, 9] if add_generation_prompt else [])


class FixedCap:
    """A cap controller with a fixed cap (the interface the loops read: cap, p, update)."""

    def __init__(self, cap):
        self.cap, self.p, self.updates = cap, 0.5, 0

    def update(self, accepted, drafted):
        self.updates += 1


def _cli_args(**kw):
    base = dict(prompt="Explain paged attention.", max_new_tokens=16, no_lookup_drafts=False,
                confidence_threshold=0.0, temperature=0.0, top_p=1.0, top_k=0, seed=0, no_chat_template=False,
                no_stream=False, max_draft=None, kv_bits=0, drafter_bits=4)
    base.update(kw)
    return types.SimpleNamespace(**base)


@pytest.mark.parametrize("mode,max_draft,chat", [("dspark", 3, True), ("dspark", "auto", False),
                                                 ("dflash", None, True), ("lookup", 4, True),
                                                 ("baseline", None, False)])
def test_cli_generate(dev, models, mode, max_draft, chat):
    target, tok, d = models["dflash" if mode == "dflash" else "dspark"]
    ctok = ChatTokenizer(tok)
    args = _cli_args(mode=mode, no_chat_template=not chat)
    pieces = []
    ctrl = FixedCap(3)
    env = {"args": args, "target": target, "tok": ctok, "drafter": d if mode in ("dspark", "dflash") else None,
           "max_draft": max_draft, "_emit": pieces.append, "calibrate": lambda *a, **k: ctrl,
           "target_repo": "synthetic/tiny", "drafter_repo": "synthetic/tiny"}
    print(f"cli generate mode={mode} max_draft={max_draft} chat={chat}", flush=True)
    made, _ = replay("cmd_generate", env, provided={"args", "target", "tok", "drafter", "_"})
    gens = [r["callee"] for r, _ in made if r["callee"].endswith("_generate")]
    assert gens == [{"dspark": "speculative_generate", "dflash": "dflash_generate", "lookup": "lookup_generate",
                     "baseline": "greedy_generate"}[mode]]
    res = env["res"]
    if max_draft == "auto":
        assert env["cap_controller"] is ctrl and ctrl.updates == res.num_rounds - res.lookup_rounds
    prompt_ids = (ctok.apply_chat_template([{"role": "user", "content": args.prompt}]) if chat
                  else ctok.encode(args.prompt))
    assert res.num_tokens >= args.max_new_tokens
    check_greedy_stream(target.model, prompt_ids, res.token_ids, MIN_MATCH)
    assert "".join(pieces) == res.text                    # everything streamed, once, in order


def test_cli_benchmark(dev, models):
    args = _cli_args(max_new_tokens=12)
    prompt = "Summarise the speculative round."
    for mode, cap in [(None, None), ("lookup", None), ("dspark", "2"), ("dspark", "auto"), ("dflash", "3")]:
        target, tok, d = models["dflash" if mode == "dflash" else "dspark"]
        ctrl = FixedCap(2)
        env = {"args": args, "target": target, "tok": tok, "drafter": d, "p": prompt, "mode": mode, "cap": cap,
               "calibrate": lambda *a, **k: ctrl, "target_repo": "synthetic/tiny", "drafter_repo": "synthetic/tiny"}
        # a run inside the mode loop, or (mode None) the baseline run before it
        in_loop = lambda r: any(next(iter(c)) == "for" for c in r["conditions"])
        sel = (lambda r: in_loop(r)) if mode else (lambda r: not in_loop(r) and r["line"] > 330)
        made, _ = replay("cmd_benchmark", env, provided={"args", "target", "tok", "drafter", "_"}, select=sel)
        runs = [(r, res) for r, res in made if r["callee"].endswith("_generate")]
        want = {None: "greedy_generate", "lookup": "lookup_generate", "dspark": "speculative_generate",
                "dflash": "dflash_generate"}[mode]
        assert [r["callee"] for r, _ in runs] == [want], (mode, cap, [r["callee"] for r, _ in runs])
        res = runs[0][1]
        print(f"cli benchmark {mode or 'baseline'} cap={cap}: {res.num_tokens} tokens, accept "
              f"{res.mean_accept_len:.2f}", flush=True)
        check_greedy_stream(target.model, tok.encode(prompt), res.token_ids, MIN_MATCH)
