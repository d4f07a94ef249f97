"""Write tests/golden/attention_s256_d768_h12.json from the reference's committed device log.

Source: /root/reference/tests/gvsoc/attention/last_run.log (runwangdl/softhier-mlir), the output of
`tests/gvsoc/run.py attention` with shape.h SEQ=256 D_MODEL=768 N_HEADS=12 CLUSTER=SH_ALL NSAMPLES=256:
256 "O0 r c hex" samples (head 0 columns, LCG seed 301) and 256 "O r c hex" samples (all columns, seed 302) of
o = softmax(q k^T / 8) v with q, k, v = lcg.fill_fp16 seeds 21 / 22 / 23 (tests/gvsoc/attention/main.c:21-23).
Only the sample lines and the config are kept (data); the log is read as text, nothing is imported.

    python tests/golden/make_attention_fixture.py [path/to/last_run.log]
"""
import json
import re
import sys
from pathlib import Path

SRC = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/gvsoc/attention/last_run.log")
OUT = Path(__file__).with_name("attention_s256_d768_h12.json")

samples = {"O0": [], "O": []}
roi = None
for ln in SRC.read_text().splitlines():
    m = re.match(r"^(O0|O) (\d+) (\d+) ([0-9a-fA-F]{4})$", ln.strip())
    if m:
        samples[m.group(1)].append([int(m.group(2)), int(m.group(3)), m.group(4).lower()])
    m = re.match(r"\[Performance Counter\]: Execution period is (\d+) ns", ln)
    if m:
        roi = int(m.group(1))
fixture = {
    "source": "runwangdl/softhier-mlir tests/gvsoc/attention/last_run.log",
    "config": {"S": 256, "D": 768, "H": 12, "dh": 64, "scale": 0.125, "seeds": {"q": [21, -8, 8, 0.125], "k": [22, -8, 8, 0.125],
               "v": [23, -16, 16, 0.125]}, "dump_seeds": {"O0": 301, "O": 302}, "nsamples": 256,
               "device": "SoftHier GVSoC, RedMulE fp16 accumulation", "reference_tolerance": {"atol": 0.05, "rtol": 0.05}},
    "roi_ns": roi,
    "samples": samples,
}
OUT.write_text(json.dumps(fixture, indent=1))
print(f"wrote {OUT}: {len(samples['O0'])} O0 + {len(samples['O'])} O samples, roi {roi} ns")
