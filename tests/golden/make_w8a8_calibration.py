"""Write hackathon_amd/calibration/decoder_w8a8.json: per-tensor activation scales.

The W8A8 decoder (12 layers, d768, 12 heads, FFN 3072, vocab 32000, S1024,
B16) needs one scale per QuantizeLinear input and per QLinearMatMul output.
They come from a float forward of the first sample with every QDQ pair
bypassed (oracle.graph_ref.calibration_ranges): scale = max|x| / 127.
The result is committed as data, so building the model never runs this
forward and the product never imports the oracle.

    python tests/golden/make_w8a8_calibration.py [--config decoder_w8a8]
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))


class _UnitScales(dict):
    """Every scale 1.0: the calibration forward bypasses quantization anyway."""

    def __missing__(self, key):
        return 1.0

    def __contains__(self, key):
        return True


def main() -> None:
    from hackathon_amd import models
    from oracle import graph_ref

    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="decoder_w8a8")
    args = ap.parse_args()
    t0 = time.time()
    m = models.build(args.config, act_scales=_UnitScales())
    first = {k: v[:1] for k, v in m.inputs.items()}
    ranges = graph_ref.calibration_ranges(m.graph, m.weights, first)
    scales = {n: max(float(ranges[n]), 1e-8) / 127.0 for n in m.meta["quant_scales"]}
    out = models.calibration_path(m.name)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps({"signature": m.meta["signature"], "method": "max|x|/127, first sample, QDQ bypassed",
                               "scales": scales}, indent=1, sort_keys=True))
    print(f"wrote {out} ({len(scales)} scales) in {time.time() - t0:.1f}s")


if __name__ == "__main__":
    main()
