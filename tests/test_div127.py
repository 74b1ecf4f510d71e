"""The Q8_0 block scale amax / 127 as the device computes it (div127 in
sam.cpp_amd/csrc/q8stage.hpp: q = x * fl(1/127), e = fma(-q, 127, x),
q' = fma(e, fl(1/127), q), +inf passed through) against IEEE division, for
every non-negative float: ggml's from_float divides (d = amax / 127), so the
stored fp16 scale must come from the correctly rounded quotient.  The check
runs as a small C program (IEEE fmaf, no contraction), about 40 s."""

import shutil
import subprocess
import textwrap

import pytest

SOURCE = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    static float div127(float x) {
        const float r = 1.0f / 127.0f;
        const float q = x * r;
        const float e = fmaf(-q, 127.0f, x);
        const float q2 = fmaf(e, r, q);
        return x < INFINITY ? q2 : x;
    }
    int main(void) {
        unsigned long long bad = 0;
        for (uint64_t b = 0; b <= 0x7f800000u; ++b) {
            const uint32_t u = (uint32_t)b;
            float x;
            memcpy(&x, &u, 4);
            volatile float ref = x / 127.0f;
            const float got = div127(x);
            uint32_t a, c;
            const float rr = ref;
            memcpy(&a, &rr, 4);
            memcpy(&c, &got, 4);
            bad += a != c;
        }
        printf("%llu\n", bad);
        return 0;
    }
""")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div127_matches_ieee_division_for_every_nonnegative_float(tmp_path):
    src = tmp_path / "div127.c"
    exe = tmp_path / "div127"
    src.write_text(SOURCE)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout
    assert int(out.strip()) == 0


def test_div127_source_matches_the_device_form():
    """The replayed steps are the device function's."""
    import pathlib
    hpp = (pathlib.Path(__file__).resolve().parents[1] / "sam.cpp_amd" / "csrc" / "q8stage.hpp").read_text()
    body = hpp[hpp.index("float div127(float x)"):]
    body = body[:body.index("}")]
    for step in ("const float r = 1.0f / 127.0f;", "const float q = x * r;",
                 "__builtin_fmaf(-q, 127.0f, x)", "__builtin_fmaf(e, r, q)", "return x < __builtin_inff() ? q2 : x;"):
        assert step in body, step
