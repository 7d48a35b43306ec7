"""Regenerate randn_prefix.json from the built host library."""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "mynah-asr_amd"))
import mynah_hip  # noqa: E402

lib = mynah_hip.HipLib()
out = [{"seed": s, "sigma": g, "values": [float(v) for v in lib.randn(s, g, (16,))]}
       for s, g in [(0, 0.02), (1, 1.0), (12345, 3.0)]]
json.dump(out, open(os.path.join(HERE, "randn_prefix.json"), "w"), indent=1)
