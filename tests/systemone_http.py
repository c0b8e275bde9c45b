"""The HTTP face of the reference's unchanged Python layer, restated as test
infrastructure (TEST CODE ONLY: nothing in the product imports it).

A drop-in user keeps running the reference's own server
(python/cujev/server.py) and decision layer (python/cujev/systemone.py) over
this build's libcujev.so. Neither can run here, so this module restates
what they ask of the engine, on the wire format they serve:

  POST /v1/systemone  {state, model, questions: {id: {type, instructions,
                      criteria}}} -> {model, answers: {id: answer}, usage:
                      {input_tokens, output_tokens}}, with the timing headers
                      x-cujev-prefill-ms / -eval-ms / -wall-ms and
                      x-cujev-prefix-cached (server.py:66-92);
  422                 {"detail": [{"loc", "msg", "type"}]} for a request that
                      fails validation (server.py:21-24, systemone.py:98-156);
  401                 when an API key is set and the Bearer header does not
                      match (server.py:42-50);
  GET /health, GET /v1/models (server.py:52-64).

The prompt layer is replaced by a character tokenizer of this file's own
(the engine never sees text: only the prefix ids, the suffix ids and the
label ids, which the reference takes from verified single-token label sets,
prompt.py:52-74). Answers, packing and the prefix cache come from
tests/systemone_caller.py, whose functions restate systemone.py:131-194;
probabilities are rounded to 4 digits as there (:67-68).
"""
from __future__ import annotations

import json
import threading
import time
from typing import Any

import numpy as np
from fastapi import FastAPI, Header, Request
from fastapi.responses import JSONResponse

from systemone_caller import confidence, pack_plan, softmax64

ALIASES = ("jev-latest", "cujev-latest")


class RequestError(ValueError):
    def __init__(self, loc, msg):
        super().__init__(msg)
        self.loc, self.msg = loc, msg


def validation_error(loc, msg, typ="value_error"):
    return JSONResponse(status_code=422,
                        content={"detail": [{"loc": loc, "msg": msg, "type": typ}]})


class CharPrompts:
    """Text -> token ids, one id per character (16 + code point mod 3000),
    and single-token labels: 'A'.., '0'..'9', and 'yes' / 'no' as two ids of
    their own above the character range."""

    YES, NO = 3100, 3101

    def encode(self, text: str) -> list[int]:
        return [16 + ord(ch) % 3000 for ch in text]

    def _label(self, s: str) -> int:
        return self.encode(s)[0]

    def prefix(self, state: Any) -> list[int]:
        text = state if isinstance(state, str) else json.dumps(state, sort_keys=True)
        return self.encode("STATE\n" + text + "\n")

    def choice(self, instructions, criteria: dict) -> tuple[list[int], list[int]]:
        labels = [chr(ord("A") + i) if i < 26 else chr(ord("a") + i - 26)
                  for i in range(len(criteria))]
        lines = [f"Q {instructions}"] + [f"{lab} {name}" for lab, name in zip(labels, criteria)]
        return self.encode("\n".join(lines) + "\n>"), [self._label(l) for l in labels]

    def score(self, instructions, levels: list) -> tuple[list[int], list[int]]:
        lines = [f"Q {instructions}"] + [f"{i} {lv}" for i, lv in enumerate(levels)]
        return self.encode("\n".join(lines) + "\n>"), [self._label(str(i))
                                                       for i in range(len(levels))]

    def noul(self, instructions, criteria) -> tuple[list[int], list[int]]:
        return self.encode(f"Q {instructions}\nyes/no\n>"), [self.YES, self.NO]


def _r(x):
    return float(round(float(x), 4))


class Layer:
    """The decision layer's request path over one engine."""

    def __init__(self, engine, branch_cls, name="cujev/test-model"):
        self.engine, self.Branch = engine, branch_cls
        self.name = name
        self.prompts = CharPrompts()
        self.lock = threading.Lock()
        self.cached = None
        self.calls = []  # branch count and tokens of every eval call

    def resolve_model(self, model):
        if not isinstance(model, str) or not model:
            raise RequestError(["body", "model"], "model must be a non-empty string")
        m = model.strip()
        if m in ALIASES or m == self.name or m.startswith("cujev"):
            return self.name
        raise RequestError(["body", "model"], f"unknown model {model!r}")

    def build(self, qid, q):
        loc = ["body", "questions", qid]
        if not isinstance(q, dict):
            raise RequestError(loc, "question must be an object")
        kind, instr, crit = q.get("type"), q.get("instructions"), q.get("criteria")
        if instr is None or (isinstance(instr, str) and not instr.strip()):
            raise RequestError(loc + ["instructions"], "instructions are required")
        if kind == "choice":
            if not isinstance(crit, dict) or not crit or len(crit) > 52:
                raise RequestError(loc + ["criteria"], "choice needs 1-52 options")
            toks, cands = self.prompts.choice(instr, crit)
            return toks, cands, ("choice", list(crit))
        if kind == "score":
            if not isinstance(crit, list) or not 2 <= len(crit) <= 10:
                raise RequestError(loc + ["criteria"], "score needs 2-10 levels")
            toks, cands = self.prompts.score(instr, crit)
            return toks, cands, ("score", list(crit))
        if kind == "noul":
            if crit is not None and not isinstance(crit, dict):
                raise RequestError(loc + ["criteria"], "noul criteria must be an object")
            toks, cands = self.prompts.noul(instr, crit)
            return toks, cands, ("noul", None)
        raise RequestError(loc + ["type"], "type must be one of choice, score, noul")

    def evaluate(self, state, model, questions):
        served = self.resolve_model(model)
        if state is None:
            raise RequestError(["body", "state"], "state is required")
        if not isinstance(questions, dict) or not questions:
            raise RequestError(["body", "questions"], "questions must be a non-empty object")
        prefix = self.prompts.prefix(state)
        if len(prefix) > self.engine.max_state_tokens:
            raise RequestError(["body", "state"], f"state is {len(prefix)} tokens")
        built = [(str(qid),) + self.build(str(qid), q) for qid, q in questions.items()]
        if max(len(b[1]) for b in built) > self.engine.max_branch_tokens:
            raise RequestError(["body", "questions"], "a question is too long")
        with self.lock:
            hit = self.cached == prefix
            prefill_ms = 0.0
            if not hit:
                self.engine.prefill(prefix)
                self.cached = prefix
                prefill_ms = self.engine.last_timing().prefill_ms
            branches = [self.Branch(toks, cands) for _, toks, cands, _ in built]
            logits, eval_ms = [], 0.0
            for a, b in pack_plan([len(x[1]) for x in built], self.engine.max_branches,
                                  self.engine.max_branch_tokens):
                logits.extend(self.engine.eval(branches[a:b]))
                eval_ms += self.engine.last_timing().eval_ms
                self.calls.append((b - a, sum(len(x[1]) for x in built[a:b])))
        answers = {}
        for (qid, _, _, (kind, opts)), lg in zip(built, logits):
            p = softmax64(lg)
            if kind == "noul":
                answers[qid] = {"type": "noul", "noul": _r(p[0])}
            elif kind == "choice":
                answers[qid] = {"type": "choice", "choice": opts[int(p.argmax())],
                                "probabilities": {o: _r(p[i]) for i, o in enumerate(opts)},
                                "confidence": _r(confidence(p))}
            else:
                answers[qid] = {"type": "score", "score": _r(np.sum(p * np.arange(len(p)))),
                                "legend": {str(i): lv for i, lv in enumerate(opts)},
                                "probabilities": {str(i): _r(v) for i, v in enumerate(p)},
                                "confidence": _r(confidence(p))}
        usage = {"input_tokens": len(prefix) + sum(len(x[1]) for x in built),
                 "output_tokens": sum(len(lg) for lg in logits)}
        return served, answers, usage, prefill_ms, eval_ms, hit


def create_app(layer: Layer, api_key: str | None = None) -> FastAPI:
    app = FastAPI()

    def auth(header):
        if api_key is None:
            return None
        if not header or not header.startswith("Bearer ") or header[7:].strip() != api_key:
            return JSONResponse(status_code=401, content={"detail": {
                "error_type": "authentication_error", "message": "Missing or invalid API key."}})
        return None

    @app.get("/health")
    def health():
        e = layer.engine
        return {"status": "ok", "model": layer.name, "engine": e.name, "version": e.version,
                "max_state_tokens": e.max_state_tokens, "max_branch_tokens": e.max_branch_tokens,
                "max_branches": e.max_branches}

    @app.get("/v1/models")
    def models(authorization: str | None = Header(default=None)):
        if (r := auth(authorization)) is not None:
            return r
        return {"models": [{"name": n} for n in (layer.name,) + ALIASES]}

    @app.post("/v1/systemone")
    async def systemone(request: Request, authorization: str | None = Header(default=None)):
        if (r := auth(authorization)) is not None:
            return r
        try:
            body = await request.json()
        except Exception:
            return validation_error(["body"], "request body must be JSON", "json_invalid")
        if not isinstance(body, dict):
            return validation_error(["body"], "request body must be an object")
        for k in ("state", "model", "questions"):
            if k not in body:
                return validation_error(["body", k], "field required", "missing")
        t0 = time.perf_counter()
        try:
            served, answers, usage, pms, ems, hit = layer.evaluate(
                body["state"], body["model"], body["questions"])
        except RequestError as e:
            return validation_error(e.loc, e.msg)
        wall = (time.perf_counter() - t0) * 1000
        return JSONResponse(
            content={"model": served, "answers": answers, "usage": usage},
            headers={"x-cujev-prefill-ms": f"{pms:.2f}", "x-cujev-eval-ms": f"{ems:.2f}",
                     "x-cujev-wall-ms": f"{wall:.2f}",
                     "x-cujev-prefix-cached": "1" if hit else "0"})

    return app
