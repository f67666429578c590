"""The north star's literal bar, |gpu - cpu| <= 1e-6 + 1e-5 |cpu|, where a test asserts a wider,
scale-aware bar instead (sums whose fp32 value depends on the order of the additions: the
LayerNorm dweight/dbias column sums, the softmax row sum). Those tests record here the fraction
of outputs inside the literal bar; it is printed and, when the environment variable
UGK_LITERAL_BAR_JSON names a file, written there as JSON at the end of the pytest session."""
import json
import os

_fractions = {}


def record(key, fraction):
    _fractions[key] = round(float(fraction), 6)
    print(f"literal-bar pass fraction, {key}: {fraction:.6f}")


def write():
    path = os.environ.get("UGK_LITERAL_BAR_JSON")
    if path and _fractions:
        with open(path, "w") as f:
            json.dump(_fractions, f, indent=1, sort_keys=True)
