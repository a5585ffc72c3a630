"""Per-layer activation formats (bits, f) for the 12 sites of a block.

The rule is python/intref.py:154-160: a site flagged in scaling_proposal.json is INT32
with f = 31 - k in wide mode, every other site is INT16 with f = 15 - k.  The fm record
of a layer lists (bits, f) for SITES in order (python/export_vectors.py:34-38).
data/fm_wide.json holds the table this rule yields for the reference's
results/scaling_proposal.json, so the package needs no copy of that file.

Run as `python -m eii.formats PROPOSAL_JSON` to regenerate data/fm_wide.json.
"""
import json
import os
import sys

from .modelbin import NL, SITES

_DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "fm_wide.json")


def fmt_from_entry(entry, wide=True):
    """(bits, f) for one proposal entry {"class": ..., "k": ...}."""
    flagged = entry["class"].startswith("flagged")
    k = int(entry["k"])
    if flagged and wide:
        return 32, 31 - k
    return 16, 15 - k


def fm_from_proposal(path, wide=True):
    """(fm [NL][24], f_y) from a scaling_proposal.json."""
    with open(path) as f:
        sites = json.load(f)["sites"]
    fm = []
    for l in range(NL):
        row = []
        for s in SITES:
            row += list(fmt_from_entry(sites[f"{s}|{l}"], wide))
        fm.append(row)
    f_y = 15 - int(sites["final_out|30"]["k"])
    return fm, f_y


def load_fm():
    """The committed wide-mode table: (fm [NL][24], f_y)."""
    with open(_DATA) as f:
        d = json.load(f)
    return d["fm"], d["f_y"]


if __name__ == "__main__":
    fm, f_y = fm_from_proposal(sys.argv[1])
    os.makedirs(os.path.dirname(_DATA), exist_ok=True)
    with open(_DATA, "w") as f:
        json.dump({"rule": "flagged & wide -> (32, 31-k) else (16, 15-k); sites in fm order",
                   "sites": list(SITES), "f_y": f_y, "fm": fm}, f, indent=0)
    print("wrote", _DATA)
