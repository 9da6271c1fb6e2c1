"""Records the public method signatures of the reference's TNNCuda<T>
(source/nncuda.pas:100-157) as data: kind, name, and each parameter's
modifier, name, type and default, in order (tests/pascal_sig.py parses them).
The signature test of pascal/nnhip.pas compares TNNHip<T> against this file.

Run (in a container that has the reference checkout):
  python tests/golden/make_tnncuda_signatures.py /root/reference/source/nncuda.pas
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from pascal_sig import parse_methods  # noqa: E402


def main(path):
    lines = open(path, encoding="utf-8", errors="replace").read().splitlines()
    region = "\n".join(lines[99:157])  # nncuda.pas:100-157, the public methods
    methods = parse_methods(region)
    assert methods[0]["name"] == "deviceCount" and methods[-1]["name"] == "loadCUBinFile", (methods[0], methods[-1])
    with open(os.path.join(HERE, "tnncuda_signatures.json"), "w") as f:
        json.dump({"source": "nncuda.pas:100-157", "methods": methods}, f, indent=1)
        f.write("\n")
    print(f"{len(methods)} methods")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/source/nncuda.pas")
