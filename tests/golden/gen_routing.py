"""Record what the reference's ``build_param_groups`` returns for each call in
``routing_cases.CASES`` (routing.py:512-789, config.py:83-108).

Run ONLY in the build container, where the reference is mounted read-only:

    python tests/golden/gen_routing.py /root/reference

The builder is pure host logic with no closed form to check it against, so its
outputs on these small models are recorded here: group names, parameter
membership by qualified name, every option, warnings and errors.  Nothing of the
reference is stored except these outcomes.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import routing_cases  # noqa: E402


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    import adafactor8bit  # the reference package
    assert os.path.abspath(adafactor8bit.__file__).startswith(os.path.abspath(ref)), adafactor8bit.__file__
    out = [routing_cases.describe(adafactor8bit.build_param_groups, m, kw) for m, kw in routing_cases.CASES]
    with open(os.path.join(HERE, "routing_groups.json"), "w") as f:
        json.dump({"cases": len(out), "outcomes": out}, f, separators=(",", ":"), sort_keys=True)
    print(f"wrote {len(out)} outcomes")


if __name__ == "__main__":
    main()
