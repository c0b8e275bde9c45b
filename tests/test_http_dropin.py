"""HTTP conformance of the drop-in: the reference's /v1/systemone wire format
(python/cujev/server.py:21-92) and request path (python/cujev/systemone.py:
98-194), restated in tests/systemone_http.py, served over an engine.

CPU tests drive the restated server over a recording stand-in engine: status
codes and error bodies, auth, headers, usage counts, the prefix cache and
packing under the engine's budgets. The GPU test serves this build's Engine
(libcujev.so) on a seeded tiny checkpoint and checks that every answer is
the one the engine's own candidate logits give.
"""
from dataclasses import dataclass

import numpy as np
import pytest

pytest.importorskip("fastapi")
pytest.importorskip("httpx")
from fastapi.testclient import TestClient  # noqa: E402

from systemone_caller import confidence, softmax64  # noqa: E402
from systemone_http import Layer, create_app  # noqa: E402


@dataclass
class FakeBranch:
    tokens: list
    candidates: list


@dataclass
class FakeTiming:
    prefill_ms: float
    eval_ms: float


class FakeEngine:
    """Candidate logits that depend on the prefix and the branch tokens, so a
    wrong prefix or a mixed-up branch shows in the answers."""

    name, version = "fake", "0.0"

    def __init__(self, mst=400, mbt=120, mb=3):
        self.max_state_tokens, self.max_branch_tokens, self.max_branches = mst, mbt, mb
        self.prefills, self.evals, self.prefix = 0, [], None

    def prefill(self, ids):
        self.prefills += 1
        self.prefix = list(ids)

    def eval(self, branches):
        assert len(branches) <= self.max_branches
        assert sum(len(b.tokens) for b in branches) <= self.max_branch_tokens
        self.evals.append(len(branches))
        return [self.logits(self.prefix, b) for b in branches]

    @staticmethod
    def logits(prefix, b):
        h = (sum(prefix) * 31 + sum(b.tokens)) % 9973
        return np.array([((h * (c + 7)) % 101) / 25.0 for c in b.candidates], np.float32)

    def last_timing(self):
        return FakeTiming(1.5, 0.5)


REQ = {
    "state": {"hp": 12, "enemies": ["orc", "bat"], "note": "door is locked"},
    "model": "jev-latest",
    "questions": {
        "flee": {"type": "noul", "instructions": "Should the player flee?"},
        "act": {"type": "choice", "instructions": "Next action",
                "criteria": {"attack": "hit the orc", "heal": "drink", "wait": "do nothing"}},
        "risk": {"type": "score", "instructions": "Danger level", "criteria": ["low", "mid", "high", "fatal"]},
        "door": {"type": "noul", "instructions": "Is the door open?",
                 "criteria": {"true": "open", "false": "closed"}},
    },
}


def client(engine, branch=FakeBranch, api_key=None):
    layer = Layer(engine, branch)
    return TestClient(create_app(layer, api_key=api_key)), layer


def test_validation_errors_have_the_reference_shape():
    c, _ = client(FakeEngine())
    cases = [
        (b"not json", ["body"], "json_invalid"),
        ([1, 2], ["body"], "value_error"),
        ({"state": 1, "model": "jev-latest"}, ["body", "questions"], "missing"),
        (dict(REQ, model="gpt-9"), ["body", "model"], "value_error"),
        (dict(REQ, state=None), ["body", "state"], "value_error"),
        (dict(REQ, questions={}), ["body", "questions"], "value_error"),
        (dict(REQ, questions={"q": {"type": "choice", "instructions": "x", "criteria": {}}}),
         ["body", "questions", "q", "criteria"], "value_error"),
        (dict(REQ, questions={"q": {"type": "score", "instructions": "x", "criteria": ["one"]}}),
         ["body", "questions", "q", "criteria"], "value_error"),
        (dict(REQ, questions={"q": {"type": "noul", "instructions": " "}}),
         ["body", "questions", "q", "instructions"], "value_error"),
        (dict(REQ, questions={"q": {"type": "vote", "instructions": "x"}}),
         ["body", "questions", "q", "type"], "value_error"),
        (dict(REQ, state="s" * 500), ["body", "state"], "value_error"),
    ]
    for body, loc, typ in cases:
        r = c.post("/v1/systemone", content=body) if isinstance(body, bytes) else \
            c.post("/v1/systemone", json=body)
        assert r.status_code == 422, (loc, r.text)
        (d,) = r.json()["detail"]
        assert d["loc"] == loc and d["type"] == typ and isinstance(d["msg"], str)


def test_auth_models_health():
    eng = FakeEngine()
    c, _ = client(eng, api_key="k1")
    assert c.post("/v1/systemone", json=REQ).status_code == 401
    assert c.post("/v1/systemone", json=REQ, headers={"Authorization": "Bearer k2"}).status_code == 401
    assert c.get("/v1/models").status_code == 401
    assert c.post("/v1/systemone", json=REQ, headers={"Authorization": "Bearer k1"}).status_code == 200
    names = [m["name"] for m in c.get("/v1/models", headers={"Authorization": "Bearer k1"}).json()["models"]]
    assert "jev-latest" in names
    h = c.get("/health").json()
    assert h["status"] == "ok" and h["max_branches"] == eng.max_branches


def test_answers_usage_headers_and_prefix_cache():
    eng = FakeEngine(mbt=120, mb=3)
    c, layer = client(eng)
    r = c.post("/v1/systemone", json=REQ)
    assert r.status_code == 200
    body = r.json()
    assert body["model"] == layer.name and set(body["answers"]) == set(REQ["questions"])
    assert r.headers["x-cujev-prefix-cached"] == "0"
    for h in ("x-cujev-prefill-ms", "x-cujev-eval-ms", "x-cujev-wall-ms"):
        float(r.headers[h])
    # every answer is the one the engine's logits give
    prefix = layer.prompts.prefix(REQ["state"])
    for qid, q in REQ["questions"].items():
        toks, cands, (kind, opts) = layer.build(qid, q)
        p = softmax64(FakeEngine.logits(prefix, FakeBranch(toks, cands)))
        a = body["answers"][qid]
        assert a["type"] == kind
        if kind == "noul":
            assert a["noul"] == pytest.approx(p[0], abs=1e-4)
        elif kind == "choice":
            assert a["choice"] == opts[int(p.argmax())]
            assert a["confidence"] == pytest.approx(confidence(p), abs=1e-4)
            assert sum(a["probabilities"].values()) == pytest.approx(1.0, abs=5e-4)
        else:
            assert a["score"] == pytest.approx(float(np.sum(p * np.arange(len(p)))), abs=1e-4)
            assert list(a["legend"].values()) == q["criteria"]
    usage = body["usage"]
    branch_tokens = sum(len(layer.build(k, q)[0]) for k, q in REQ["questions"].items())
    assert usage == {"input_tokens": len(prefix) + branch_tokens, "output_tokens": 2 + 3 + 4 + 2}
    # packing under the budgets, then the prefix cache on a repeat
    assert eng.prefills == 1 and len(eng.evals) >= 2 and max(eng.evals) <= 3
    r2 = c.post("/v1/systemone", json=REQ)
    assert r2.headers["x-cujev-prefix-cached"] == "1" and eng.prefills == 1
    assert r2.json()["answers"] == body["answers"]
    r3 = c.post("/v1/systemone", json=dict(REQ, state={"hp": 3}))
    assert r3.headers["x-cujev-prefix-cached"] == "0" and eng.prefills == 2


@pytest.mark.gpu
def test_http_over_this_engine(tmp_path):
    """The restated server over libcujev.so: answers equal the engine's own
    candidate logits' answers, the repeat hits the prefix cache with the same
    answers, and the headers carry the engine's timings."""
    pytest.importorskip("torch")
    from cujev import Branch, Engine, synthetic

    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    synthetic.write_checkpoint(tmp_path, cfg, seed=8, norm_std=0.1)
    with Engine(str(tmp_path), max_state_tokens=512, max_branch_tokens=96, max_branches=2) as e:
        c, layer = client(e, Branch)
        r = c.post("/v1/systemone", json=REQ)
        assert r.status_code == 200, r.text
        body = r.json()
        assert float(r.headers["x-cujev-prefill-ms"]) > 0 and float(r.headers["x-cujev-eval-ms"]) > 0
        assert len(layer.calls) >= 2 and all(n <= 2 and t <= 96 for n, t in layer.calls)
        prefix = layer.prompts.prefix(REQ["state"])
        built = {k: layer.build(k, q) for k, q in REQ["questions"].items()}
        direct = e.eval([Branch(t, cd) for t, cd, _ in built.values()][:2])  # same prefix state
        for (qid, (toks, cands, (kind, opts))), lg in zip(list(built.items())[:2], direct):
            p = softmax64(lg)
            a = body["answers"][qid]
            if kind == "noul":
                assert a["noul"] == pytest.approx(p[0], abs=3e-3)
            else:
                assert a["probabilities"][opts[0]] == pytest.approx(p[0], abs=3e-3)
        r2 = c.post("/v1/systemone", json=REQ)
        assert r2.headers["x-cujev-prefix-cached"] == "1"
        assert r2.json()["answers"] == body["answers"]
        print(f"http over the engine: {len(layer.calls)} eval calls, input tokens "
              f"{body['usage']['input_tokens']} (prefix {len(prefix)})")
