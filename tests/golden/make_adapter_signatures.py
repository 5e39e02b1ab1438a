"""Writes tests/golden/adapter_signatures.json: the interface this backend must
match, taken from the reference's Lua text (read, not run).

For every `function M.<name>(<params>)` and `function Handle:<name>(<params>)`
of ai/gpu/luatl_adapter.lua, and every `function Prog:<name>(<params>)` of
luaTL.Program (ai/gpu/luaTL_train.lua:332-632), the name and parameter list,
plus the module fields the adapter sets.  Only names and parameter lists are
recorded: the interface, not the code.

    python tests/golden/make_adapter_signatures.py [/root/reference]
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def signatures(text, owner):
    pat = re.compile(r"^function\s+" + re.escape(owner) + r"([.:])(\w+)\s*\(([^)]*)\)", re.M)
    out = {}
    for m in pat.finditer(text):
        params = [p.strip() for p in m.group(3).split(",") if p.strip()]
        out[m.group(2)] = params
    return out


def main(ref):
    adapter = open(os.path.join(ref, "ai", "gpu", "luatl_adapter.lua")).read()
    train = open(os.path.join(ref, "ai", "gpu", "luaTL_train.lua")).read()
    ctor = re.search(r"local M\s*=\s*\{([^}]*)\}", adapter).group(1)
    fields = sorted(set(re.findall(r"\bM\.(\w+)\s*=[^=]", adapter)) | set(re.findall(r"(\w+)\s*=", ctor)))
    data = {
        "source": {"adapter": "ai/gpu/luatl_adapter.lua", "program": "ai/gpu/luaTL_train.lua:332-632"},
        "module": signatures(adapter, "M"),
        "handle": signatures(adapter, "Handle"),
        "program": signatures(train, "Prog"),
        "fields": fields,
    }
    with open(os.path.join(HERE, "adapter_signatures.json"), "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{len(data['module'])} module functions, {len(data['handle'])} handle methods, "
          f"{len(data['program'])} program methods, fields {fields}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
