"""Writes var_dump_expectations.json: the values printed in the --EXPECT--
blocks of reference tests that report results with var_dump (arithmetic
with broadcasting, where, prod, transfers).  Each block becomes a list of
entries, either {"value": ...} for one var_dump (arrays as nested lists,
floats as numbers, with "nan"/"inf"/"-inf" spelled out) or {"text": line} for
a printed line.  The inputs themselves are restated in the tests that read
this file.  Run in a checkout that has the reference at /root/reference."""
import json
import os
import re

REF = "/root/reference/tests"
FILES = ["ca_add", "ca_add_overload", "ca_sub", "ca_sub_overload", "ca_mult", "ca_mult_overload",
         "ca_div", "ca_div_overload", "ca_where", "ca_prod_reduce", "ca_transfer"]


def parse_expect(text):
    body = text.split("--EXPECT--", 1)[1].strip("\n").splitlines()
    pos = 0

    def value():
        nonlocal pos
        line = body[pos].strip()
        pos += 1
        m = re.fullmatch(r"array\((\d+)\) \{", line)
        if m:
            n = int(m.group(1))
            items = []
            for _ in range(n):
                key = body[pos].strip()
                assert re.fullmatch(r"\[\d+\]=>", key), key
                pos += 1
                items.append(value())
            assert body[pos].strip() == "}", body[pos]
            pos += 1
            return items
        m = re.fullmatch(r"float\((.*)\)", line)
        if m:
            v = m.group(1)
            low = v.lower()
            return low if low in ("nan", "inf", "-inf") else float(v)
        m = re.fullmatch(r"int\((-?\d+)\)", line)
        if m:
            return int(m.group(1))
        m = re.fullmatch(r"bool\((true|false)\)", line)
        if m:
            return m.group(1) == "true"
        if line == "NULL":
            return None
        m = re.fullmatch(r'string\(\d+\) "(.*)"', line)
        if m:
            return {"string": m.group(1)}
        raise ValueError(f"unparsed line {line!r}")

    out = []
    while pos < len(body):
        line = body[pos].strip()
        if re.match(r"(array\(\d+\) \{|float\(|int\(|bool\(|NULL$|string\()", line):
            out.append({"value": value()})
        else:
            out.append({"text": line})
            pos += 1
    return out


def main():
    result = {"_about": "values printed by var_dump in the --EXPECT-- blocks of the named reference tests "
                        "(tests/<name>.phpt), in order"}
    for name in FILES:
        with open(os.path.join(REF, name + ".phpt")) as f:
            result[name] = parse_expect(f.read())
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "var_dump_expectations.json")
    with open(out, "w") as f:
        json.dump(result, f, indent=None, separators=(",", ":"))
        f.write("\n")


if __name__ == "__main__":
    main()
