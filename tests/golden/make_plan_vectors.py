#!/usr/bin/env python3
"""Writes tests/golden/plan_vectors.json: attention-plan tile settings recorded in the reference's
own run reports (docs/reports/*.json), as inputs (groups, tokens, heads, plan) and the tiles and
score bytes the reference reported. Run in the build container, where the reference's
documents are present; the tests read only the JSON written here.

Two sources:
* run reports with an ``effective_config`` (deux-wgpu-3s, hyperace-native-short,
  leap-native-30s, mp3-slice-3s): the time pass of the plan of their version (query tile 128,
  group tile 4, 512 MiB, one host thread) and its ``estimated_time_attention_score_bytes``;
* docs/reports/cuda-benchmark.json: the automatic tiles of both axis passes per backend
  (``BackendKind::attention_plan``: host threads as reported, no explicit tiles). Model shapes
  come from the run reports of the same model id; "native-context" runs use the model's own
  chunk, "custom-context" ("short") runs the 3 s chunk of 132300 samples
  (docs/performance.md:43).
"""
from __future__ import annotations

import json
import os
import sys

REPORTS = "/root/reference/docs/reports"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "plan_vectors.json")
SHORT_CHUNK = 132300
BUDGET = 512 << 20


def load(name):
    with open(os.path.join(REPORTS, name)) as f:
        return json.load(f)


def main() -> int:
    models, cases = {}, []
    for name in sorted(os.listdir(REPORTS)):
        if not name.endswith(".json"):
            continue
        d = load(name)
        if not isinstance(d, dict) or "bands" not in d.get("effective_config", {}):
            continue
        c = d["effective_config"]
        frames = c["chunk_samples"] // c["hop"] + 1
        shape = {"heads": c["heads"], "bands": len(c["bands"]), "hop": c["hop"]}
        if d["profile"] == "native-context":
            shape["native_chunk"] = c["chunk_samples"]
        models.setdefault(d["model_id"], {}).update(shape)
        cases.append({
            "source": f"docs/reports/{name}",
            "pass": "time", "groups": len(c["bands"]), "tokens": frames, "heads": c["heads"],
            "plan": {"query_tile": 128, "group_tile": 4, "score_budget": BUDGET,
                     "host_threads": 1},
            "want": {"group_tile": d["group_tile"], "query_tile": d["query_tile"],
                     "score_bytes": d["estimated_time_attention_score_bytes"]},
        })
    bench = load("cuda-benchmark.json")
    for entry in bench["entries"]:
        m = models.get(entry["model_id"])
        for backend, run in entry["backends"].items():
            s = run.get("settings", {})
            if "group_tile" not in s or m is None:
                continue
            chunk = m["native_chunk"] if s["profile"] == "native-context" else SHORT_CHUNK
            frames = chunk // m["hop"] + 1
            plan = {"query_tile": None, "group_tile": None, "score_budget": BUDGET,
                    "host_threads": s["host_threads"]}
            src = f"docs/reports/cuda-benchmark.json {entry['label']} {backend}"
            for axis, groups, tokens, prefix in (("time", m["bands"], frames, ""),
                                                 ("frequency", frames, m["bands"],
                                                  "frequency_")):
                cases.append({
                    "source": src, "pass": axis, "groups": groups, "tokens": tokens,
                    "heads": m["heads"], "plan": plan, "backend": backend,
                    "want": {"group_tile": s[prefix + "group_tile"],
                             "query_tile": s[prefix + "query_tile"],
                             "linear_layout": s["linear_layout"]},
                })
    with open(OUT, "w") as f:
        json.dump({"cases": cases}, f, indent=1)
        f.write("\n")
    print(f"wrote {len(cases)} cases to {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
