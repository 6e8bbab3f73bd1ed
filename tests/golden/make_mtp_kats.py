"""Write mtp_rollback_kats.json: the known-answer cases of the reference's
MtpRollbackTests (LLM/tests/MtpRollbackTests.swift:10-77), as data.

Inputs are the test's literals.  Expected values are the test's own: the
integer vectors it states (:24, :30, :57, :62) and, for the decay cases, the
formula it evaluates (:36-38, :67-75) using the outer products it lists in
its comment (:47-48), computed here in double.  Nothing here calls the oracle.
"""
import json
import math
from pathlib import Path

s0 = [1, 0, 0, 1]
k2, d2 = [1, 2, 5, 6], [3, 4, 7, 8]
k5 = [1, 2, 5, 6, 1, 1, 2, 0, 1, 1]
d5 = [3, 4, 7, 8, 1, 1, 0, 3, 2, 2]
outer5 = [[3, 4, 6, 8], [35, 40, 42, 48], [1, 1, 1, 1], [0, 6, 0, 0], [2, 2, 2, 2]]

cases = []


def add(name, m, C, k, delta, gcum, want, src):
    cases.append(dict(name=name, m=m, H=1, DK=2, DV=2, C=C, s0=s0, k=k, delta=delta,
                      gcum=gcum, want=want, source=src))


add("full_prefix_no_decay", 2, 2, k2, d2, [0, 0], [39, 44, 48, 57], "MtpRollbackTests.swift:21-25")
add("partial_prefix_no_decay", 1, 2, k2, d2, [0, 0], [4, 4, 6, 9], "MtpRollbackTests.swift:27-31")
eM, w0 = math.exp(-1.5), math.exp(-0.5)
add("decay_weighting", 2, 2, k2, d2, [-1, -1.5],
    [eM * 1 + w0 * 3 + 35, w0 * 4 + 40, w0 * 6 + 42, eM * 1 + w0 * 8 + 48],
    "MtpRollbackTests.swift:33-40")
add("m4_no_decay", 4, 5, k5, d5, [0] * 5, [40, 51, 49, 58], "MtpRollbackTests.swift:55-58")
add("m5_no_decay", 5, 5, k5, d5, [0] * 5, [42, 53, 51, 60], "MtpRollbackTests.swift:60-63")
g = [-1, -1.5, -1.8, -2.0, -2.1]
eM = math.exp(g[3])
w = [math.exp(g[3] - g[t]) for t in range(4)]
want = [eM * s0[i] + sum(w[t] * outer5[t][i] for t in range(4)) for i in range(4)]
add("m4_decay", 4, 5, k5, d5, g, want, "MtpRollbackTests.swift:65-77")

out = {"tolerance_abs": 1e-3, "tolerance_source": "MtpRollbackTests.swift:79-85",
       "cases": cases}
Path(__file__).with_name("mtp_rollback_kats.json").write_text(json.dumps(out, indent=1))
