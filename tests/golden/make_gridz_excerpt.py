"""Writes gridz_policy_excerpt.json: the keys and selected caps of the
reference's grid.z policy artefact (results/gridz_policy.json), without the
timing candidates.  Run in the build container only; the excerpt is data (the
recorded keys and their values), used to pin the key format and the lookup."""
import json
from pathlib import Path

SRC = Path("/root/reference/results/gridz_policy.json")
OUT = Path(__file__).with_name("gridz_policy_excerpt.json")

data = json.loads(SRC.read_text())
entries = {k: {"grid_z_max_layers": v["grid_z_max_layers"]} for k, v in data["entries"].items()}
OUT.write_text(json.dumps({"version": data.get("version", 1), "entries": entries}, indent=1))
print(OUT, len(entries), "entries")
