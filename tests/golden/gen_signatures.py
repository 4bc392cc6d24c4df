"""Write the positional parameter names of every function the reference's
compiled module exports (adafactor8bit/kernels.cu:3089-3150, the ``*_cuda``
host functions they bind) to ``module_signatures.json``.

    python tests/golden/gen_signatures.py /root/reference/adafactor8bit/kernels.cu
"""
import json
import os
import re
import sys


def main(path):
    src = open(path).read()
    names = re.findall(r'm\.def\("(\w+)",\s*&(\w+)\)', src)
    out = {}
    for name, fn in names:
        m = re.search(r"(?:void|torch::Tensor) " + fn + r"\((.*?)\)\s*\{", src, re.S)
        out[name] = [a.strip().split()[-1] for a in m.group(1).split(",")]
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "module_signatures.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=0)
    print(f"{len(out)} signatures -> {dst}")


if __name__ == "__main__":
    main(sys.argv[1])
