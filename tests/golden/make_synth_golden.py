"""Writes synth_normal_seed0.json: the first 64 values of kf_synth_normal(seed 0, sigma 1) as f32 bit patterns.

Regenerate with `python tests/golden/make_synth_golden.py` after building the library. The values are also checked
against an independent numpy restatement of the generator in tests/test_host_abi.py.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import kungfu_amd as kf  # noqa: E402

v = kf.synth_normal(0, 1.0, 64)
json.dump({"seed": 0, "sigma": 1.0, "bits": [int(b) for b in v.view("uint32")], "values": [float(x) for x in v]},
          open(os.path.join(HERE, "synth_normal_seed0.json"), "w"), indent=0)
