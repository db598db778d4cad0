"""Writes transfer_contract.json: the raw byte patterns (13 storage dtypes,
eight elements each) and the expected logical shapes and element indices of
the nine view layouts of the reference's transfer fixture
(tests/fixtures/transfer_contract.php:1-30).  The file is read as text; the
view recipes themselves are restated with this package's view methods in
tests/test_gpu_transfer_contract.py.  Run in a checkout that has the
reference at /root/reference."""
import json
import os
import re

SRC = "/root/reference/tests/fixtures/transfer_contract.php"


def main():
    text = open(SRC).read()
    patterns = dict(re.findall(r"'(\w+)' => '([0-9a-f]+)'", text))
    layouts = {}
    for name, shape, idx in re.findall(r"'([\w-]+)' => \[\[([0-9, ]*)\], \[([0-9, ]*)\]", text):
        layouts[name] = {"shape": [int(v) for v in shape.split(",") if v.strip()],
                         "indices": [int(v) for v in idx.split(",") if v.strip()]}
    assert len(patterns) == 13 and len(layouts) == 9, (len(patterns), len(layouts))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "transfer_contract.json")
    with open(out, "w") as f:
        json.dump({"source": "tests/fixtures/transfer_contract.php:1-30", "patterns": patterns,
                   "layouts": layouts}, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
