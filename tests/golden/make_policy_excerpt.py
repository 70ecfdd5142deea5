"""Writes policy_profile_excerpt.json: one kernel profile (its rows and the
kernel_signature the reference recorded for them) and the execution entry
keyed by that signature, taken from the reference's policy artefact
(results/hierarchical_policy.json).  Run in the build container only; the
excerpt is data (inputs and the recorded fingerprint), used to pin the
signature algorithm and the lookup rules."""
import json
from pathlib import Path

SRC = Path("/root/reference/results/hierarchical_policy.json")
OUT = Path(__file__).with_name("policy_profile_excerpt.json")

data = json.loads(SRC.read_text())
prof = data["kernel_profiles"][0]
exe = [e for e in data["execution_entries"] if e.get("kernel_signature") == prof["kernel_signature"]
       and list(e["dims"]) == list(prof["dims"]) and e["batch"] == prof["batch"]]
excerpt = {
    "schema_version": data["schema_version"],
    "kernel_profiles": [prof],
    "kernel_entries": data["kernel_entries"][:2],
    "execution_entries": [{k: v for k, v in exe[0].items() if k in ("dims", "batch", "activation", "dtype",
                                                                    "kernel_signature", "best")}] if exe else [],
}
OUT.write_text(json.dumps(excerpt, indent=1))
print(OUT, len(prof["kernel_entries"]), "rows; signature", prof["kernel_signature"], "; execution entries", len(excerpt["execution_entries"]))
