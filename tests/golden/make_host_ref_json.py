"""Extract the known-answer values of the reference's generated
tests/host_ref.h (sigma schedules for 4 (steps, seq_len) cases and 144 RoPE
table samples) into tests/golden/host_ref.json. Only the numbers are kept.

    python tests/golden/make_host_ref_json.py /root/reference/tests/host_ref.h
"""
import json
import os
import re
import sys

src = open(sys.argv[1] if len(sys.argv) > 1 else
           "/root/reference/tests/host_ref.h").read()
num = r"-?[0-9.]+(?:e-?[0-9]+)?"
sig = {int(m.group(1)): [float(x) for x in re.findall(num + "(?=f)", m.group(2))]
       for m in re.finditer(r"host_ref_sigmas_(\d+)\[\d+\] = \{([^}]*)\}", src)}
cases = [{"steps": int(a), "seq_len": int(b), "sigmas": sig[int(c)]}
         for a, b, c in re.findall(r"\{(\d+), (\d+), host_ref_sigmas_(\d+)\}", src)]
body = src[src.index("host_ref_rope_samples"):]
rope = [{"axis": int(a), "table_row": int(r), "pair": int(p),
         "cos": float(c), "sin": float(s)}
        for a, r, p, c, s in re.findall(
            r"\{(\d+), (\d+), (\d+), (" + num + r")f, (" + num + r")f\}", body)]
out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host_ref.json")
json.dump({"schedule_cases": cases, "rope_samples": rope}, open(out, "w"), indent=0)
print(len(cases), "cases", len(rope), "rope samples ->", out)
