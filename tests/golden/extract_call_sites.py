"""Extract the call sites of the reference's own callers into tests/golden/call_sites.json.

    python tests/golden/extract_call_sites.py [/root/reference]

Parses src/mlx_dspark/server.py and src/mlx_dspark/cli.py with ``ast`` (nothing is imported or
run). For each caller function listed in FUNCS it records, in line order, the statements a
replay needs:
  - "call": a call whose callee is part of the API this engine keeps (the generate loops,
    SpecSlots and its methods, the prefix store, batch_generate_baseline, the loaders,
    calibrate, the server's own _generate_impl): the callee, positional and keyword arguments
    and the names the result is assigned to (a ``for`` over the call records its targets);
  - "bind": an assignment of any other expression: "groups" holds one list of target names per
    assignment target (`a = b = v` gives [[a], [b]], `a, b = v` gives [[a, b]]);
  - "reraise": a bare ``raise`` that ends an ``except`` handler.
Records inside a handler carry the name its ``except ... as name`` binds ("handler_as").
A call whose result the function returns records the target "return".
Each record carries the conditions that reach it: the tests of the enclosing ``if`` statements
(negated in an ``else`` branch), the tests of earlier ``if ...: return`` statements (negated),
and the ``for`` loops around it; and its placement: a ``try`` body, an ``except`` handler, a
``finally`` block or the plain body. The function's parameter names are stored with it.

Values are stored in a small expression grammar (JSON objects), not as source text:
  {"name": n}  {"attr": "a.b.c"}  {"const": v}  {"or": [x, y]}  {"and": [x, y]}  {"not": x}
  {"neg": x}  {"if": [test, then, else]}  {"cmp": [left, op, right]}  {"bin": [left, op, right]}
  {"item": [x, i]}  {"call": "f.g", "args": [...], "kwargs": {...}}  {"lambda": [params], "body": x}
  {"fstr": [str | {"expr": x}, ...]}  {"for": [target, iter]}  {"unsupported": node type}
tests/test_gpu_callers.py interprets these records with a driver of its own to make the same
calls against this package."""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

API = {"speculative_generate", "dflash_generate", "greedy_generate", "lookup_generate", "SpecSlots",
       "batch_generate_baseline", "PrefixCache", "target_cache_reusable", "calibrate", "admit", "step",
       "acquire", "store", "reset", "_generate_impl", "load_target", "load_drafter", "load_dflash", "bind"}
FUNCS = {
    "src/mlx_dspark/server.py": ["Engine._build_prefix_cache", "Engine._generate_impl", "BatchEngine._admit",
                                 "BatchEngine._run_session", "BatchEngine._run_serial", "BatchEngine._run_batched"],
    "src/mlx_dspark/cli.py": ["cmd_generate", "cmd_benchmark"],
}
OPS = {ast.Eq: "==", ast.NotEq: "!=", ast.Is: "is", ast.IsNot: "is not", ast.Lt: "<", ast.LtE: "<=",
       ast.Gt: ">", ast.GtE: ">=", ast.In: "in", ast.NotIn: "not in"}
BINOPS = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.FloorDiv: "//", ast.Div: "/", ast.Mod: "%"}


def dotted(node):
    if isinstance(node, ast.Name):
        return node.id
    if isinstance(node, ast.Attribute):
        base = dotted(node.value)
        return None if base is None else f"{base}.{node.attr}"
    return None


def conv(node):
    if isinstance(node, ast.Name):
        return {"name": node.id}
    if isinstance(node, ast.Attribute):
        d = dotted(node)
        return {"attr": d} if d else {"getattr": [conv(node.value), node.attr]}
    if isinstance(node, ast.Constant):
        return {"const": node.value}
    if isinstance(node, ast.BoolOp):
        return {"or" if isinstance(node.op, ast.Or) else "and": [conv(v) for v in node.values]}
    if isinstance(node, ast.UnaryOp):
        if isinstance(node.op, ast.Not):
            return {"not": conv(node.operand)}
        if isinstance(node.op, ast.USub):
            return {"neg": conv(node.operand)}
    if isinstance(node, ast.BinOp) and type(node.op) in BINOPS:
        return {"bin": [conv(node.left), BINOPS[type(node.op)], conv(node.right)]}
    if isinstance(node, ast.IfExp):
        return {"if": [conv(node.test), conv(node.body), conv(node.orelse)]}
    if isinstance(node, ast.Compare) and len(node.ops) == 1:
        return {"cmp": [conv(node.left), OPS.get(type(node.ops[0]), "?"), conv(node.comparators[0])]}
    if isinstance(node, ast.Call):
        return {"call": dotted(node.func) or "?", "args": [conv(a) for a in node.args],
                "kwargs": {k.arg: conv(k.value) for k in node.keywords if k.arg}}
    if isinstance(node, ast.Subscript):
        return {"item": [conv(node.value), conv(node.slice)]}
    if isinstance(node, ast.Lambda):
        return {"lambda": [a.arg for a in node.args.args], "body": conv(node.body)}
    if isinstance(node, ast.JoinedStr):
        parts = []
        for v in node.values:
            if isinstance(v, ast.Constant):
                parts.append(v.value)
            elif isinstance(v, ast.FormattedValue):
                parts.append({"expr": conv(v.value)})
        return {"fstr": parts}
    if isinstance(node, ast.Tuple):
        return {"tuple": [conv(e) for e in node.elts]}
    return {"unsupported": type(node).__name__}


def find_function(tree, qual):
    nodes, found = tree.body, None
    for p in qual.split("."):
        found = next((n for n in nodes if isinstance(n, (ast.FunctionDef, ast.ClassDef)) and n.name == p), None)
        if found is None:
            raise ValueError(f"{qual}: {p} not found")
        nodes = found.body
    return found


def _targets(t):
    if isinstance(t, ast.Tuple):
        return [dotted(e) for e in t.elts]
    return [dotted(t)]


def _api_calls(node):
    """API calls inside an expression, outside nested function definitions (lambdas included)."""
    out = []
    for sub in ast.walk(node):
        if isinstance(sub, ast.Call):
            c = dotted(sub.func)
            if c is not None and c.split(".")[-1] in API:
                out.append(sub)
    return out


def _returns(stmts):
    """The block leaves what follows it: return, raise, or (in a loop body) continue / break."""
    return bool(stmts) and isinstance(stmts[-1], (ast.Return, ast.Raise, ast.Continue, ast.Break))


def records(fn, rel):
    out = []

    def emit(kind, node, conds, place, **kw):
        out.append({"kind": kind, "file": rel, "line": node.lineno, "conditions": list(conds), "placement": place,
                    **kw})

    def call_record(call, conds, place, assign):
        emit("call", call, conds, place, callee=dotted(call.func), args=[conv(a) for a in call.args],
             kwargs={k.arg: conv(k.value) for k in call.keywords if k.arg}, assign=assign)

    def visit_list(stmts, conds, place):
        """Visit statements; an `if ...: return` adds its negated test to what follows it.
        Returns the guards added (a try passes its body's guards to the statements after it)."""
        conds = list(conds)
        added = []
        for s in stmts:
            if isinstance(s, ast.If) and _returns(s.body) and not s.orelse:
                visit(s, conds, place)
                g = {"not": conv(s.test)}
                conds.append(g)
                added.append(g)
                continue
            added_here = visit(s, conds, place)
            conds += added_here
            added += added_here
        return added

    def visit(node, conds, place):
        if isinstance(node, ast.If):
            for c in _api_calls(node.test):
                call_record(c, conds, place, None)
            visit_list(node.body, conds + [conv(node.test)], place)
            visit_list(node.orelse, conds + [{"not": conv(node.test)}], place)
            return []
        if isinstance(node, ast.Try):
            # a guard that returns inside the try body (or returns from every handler) still
            # guards the statements after the try
            added = visit_list(node.body, conds, "try")
            for h in node.handlers:
                n0 = len(out)
                visit_list(h.body, conds + added, "except")
                for r in h.body:
                    if isinstance(r, ast.Raise) and r.exc is None:
                        emit("reraise", r, conds + added, "except")
                for rec in out[n0:]:
                    rec["handler_as"] = h.name      # the `except ... as name` binding, or None
            visit_list(node.orelse, conds + added, place)
            visit_list(node.finalbody, conds + added, "finally")
            return added
        if isinstance(node, ast.While):
            for c in _api_calls(node.test):
                call_record(c, conds, place, None)
            visit_list(node.body, conds + [{"while": conv(node.test)}], place)
            return []
        if isinstance(node, ast.For):
            for c in _api_calls(node.iter):
                call_record(c, conds, place, _targets(node.target) if c is node.iter else None)
            visit_list(node.body, conds + [{"for": [conv(node.target), conv(node.iter)]}], place)
            return []
        if isinstance(node, (ast.Assign, ast.AnnAssign)):
            value = node.value
            if value is None:
                return []
            targets = node.targets if isinstance(node, ast.Assign) else [node.target]
            groups = [_targets(t) for t in targets]       # `a = b = v`: two groups; `a, b = v`: one
            calls = _api_calls(value)
            for c in calls:
                call_record(c, conds, place, groups[0] if c is value else None)
            if not (calls and calls[0] is value):
                emit("bind", node, conds, place, names=[n for g in groups for n in g], groups=groups,
                     value=conv(value))
            return []
        if isinstance(node, ast.Return) and node.value is not None:
            calls = _api_calls(node.value)
            for c in calls:
                call_record(c, conds, place, ["return"] if c is node.value else None)
            return []
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)):
            return []
        for c in _api_calls(node):
            call_record(c, conds, place, None)
        return []

    visit_list(fn.body, [], "body")
    return out


def extract(ref: Path) -> list:
    funcs = []
    for rel, quals in FUNCS.items():
        tree = ast.parse((ref / rel).read_text())
        for qual in quals:
            fn = find_function(tree, qual)
            funcs.append({"function": qual, "file": rel, "line": fn.lineno, "params": [a.arg for a in fn.args.args],
                          "records": records(fn, rel)})
    return funcs


def main(argv):
    ref = Path(argv[1] if len(argv) > 1 else "/root/reference")
    funcs = extract(ref)
    out = Path(__file__).with_name("call_sites.json")
    out.write_text(json.dumps({"source": "regeter/mlx-dspark v0.3.1", "functions": funcs}, indent=1) + "\n")
    n = sum(len(f["records"]) for f in funcs)
    print(f"{len(funcs)} functions, {n} records -> {out}")


if __name__ == "__main__":
    main(sys.argv)
