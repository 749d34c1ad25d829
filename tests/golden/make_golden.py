"""Writes tests/golden/config1.json from the oracle (run: python -m tests.golden.make_golden).

The fixture pins the oracle's config-1 results against later changes: the page
tables, SHA-256 of the K/V pools after the token-by-token appends and of the
f32 attention output, and the first attention values.
"""
import hashlib
import json
import os

from tests.golden import config1

HERE = os.path.dirname(os.path.abspath(__file__))


def summary():
    steps, q, tables = config1.generate()
    kc, vc = config1.oracle_cache(steps)
    online, reference = config1.oracle_attention(kc, vc, q, tables)
    return {
        "config": "BASELINE config 1 (fp16, one layer, Hkv 8, D 128, Hq 16, 16-token pages, "
                  "lengths 37/128/513/1000, seed 0)",
        "tables": [t.tolist() for t in tables],
        "appended_rows": sum(len(s[0]) for s in steps),
        "key_pool_sha256": hashlib.sha256(kc.tobytes()).hexdigest(),
        "value_pool_sha256": hashlib.sha256(vc.tobytes()).hexdigest(),
        "query_sha256": hashlib.sha256(q.tobytes()).hexdigest(),
        "attention_online_f32_sha256": hashlib.sha256(online.tobytes()).hexdigest(),
        "attention_first_values": [float(x) for x in online.ravel()[:8]],
        "attention_reference_first_values": [float(x) for x in reference.ravel()[:8]],
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "config1.json"), "w") as fh:
        json.dump(summary(), fh, indent=1)
        fh.write("\n")
    print("wrote", os.path.join(HERE, "config1.json"))
