"""The oracle's pins have teeth: plausible mistakes, planted one at a time in a copy of oracle/v7_oracle.c
(on the CPU, in a temporary directory), must each make tests/test_oracle.py fail.

Each mutant is a mistake a restatement of the reference kernels could plausibly make: another reduction
tree or accumulator pairing, leftover blocks taken last, an unfused FMA chain or rotation, a fused or
reordered scale, a missing pos-0 branch, a quantizer without its floor or with another rounding, a wrong
scale index, a truncating or flushing binary16 conversion, an FP environment with DAZ or FTZ alone.  The AVX2 cross-check is left out (it is a
second restatement, not an independent fact), and so are the golden fixtures (written by the oracle).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")

MUTANTS = [
    ("hadd: pairs v[i]+v[i+1]",
     "    float s0 = v[0] + v[4];\n"
     "    float s1 = v[1] + v[5];\n"
     "    float s2 = v[2] + v[6];\n"
     "    float s3 = v[3] + v[7];",
     "    float s0 = v[0] + v[1];\n"
     "    float s1 = v[2] + v[3];\n"
     "    float s2 = v[4] + v[5];\n"
     "    float s3 = v[6] + v[7];"),
    ("hadd: left to right",
     "    float t0 = s0 + s1;\n"
     "    float t2 = s2 + s3;\n"
     "    return t0 + t2;",
     "    return ((s0 + s1) + s2) + s3;"),
    ("sumsq: (A+C)+(B+D)",
     "        float ab = acc[0][j] + acc[1][j];\n"
     "        float cd = acc[2][j] + acc[3][j];",
     "        float ab = acc[0][j] + acc[2][j];\n"
     "        float cd = acc[1][j] + acc[3][j];"),
    ("sumsq: leftovers last",
     "    for (; b < left; ++b)\n"
     "        for (int j = 0; j < 8; ++j)\n"
     "            acc[0][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[0][j]);\n"
     "    for (int g = 0; g < blocks / 4; ++g)\n"
     "        for (int q = 0; q < 4; ++q, ++b)\n"
     "            for (int j = 0; j < 8; ++j)\n"
     "                acc[q][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[q][j]);",
     "    for (int g = 0; g < blocks / 4; ++g)\n"
     "        for (int q = 0; q < 4; ++q, ++b)\n"
     "            for (int j = 0; j < 8; ++j)\n"
     "                acc[q][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[q][j]);\n"
     "    for (; b < blocks; ++b)\n"
     "        for (int j = 0; j < 8; ++j)\n"
     "            acc[0][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[0][j]);"),
    ("sumsq: mul+add instead of fma",
     "                acc[q][j] = fmaf(x[8 * b + j], x[8 * b + j], acc[q][j]);",
     "                acc[q][j] = acc[q][j] + x[8 * b + j] * x[8 * b + j];"),
    ("scale: rsqrt fused",
     "    float root = sqrtf(val);\n"
     "    return 1.0f / root;",
     "    return (float)(1.0 / sqrt((double)val));"),
    ("scale: eps inside mean",
     "    float mean = sumsq / (float)n;\n"
     "    float val = mean + eps;",
     "    float mean = (sumsq + eps) / (float)n;\n"
     "    float val = mean;"),
    ("scale: multiply by 1/n",
     "    float mean = sumsq / (float)n;",
     "    float mean = sumsq * (1.0f / (float)n);"),
    ("add_rmsnorm: (s*w)*x",
     "        float t = s * residual[i];\n"
     "        o[i] = t * weight[i];",
     "        float t = s * weight[i];\n"
     "        o[i] = t * residual[i];"),
    ("rope: xe*w before scale",
     "        float xe = x[j] * scale;\n"
     "        float xo = x[j + half] * scale;\n"
     "        xe = xe * w[j];\n"
     "        xo = xo * w[j + half];",
     "        float xe = x[j] * w[j];\n"
     "        float xo = x[j + half] * w[j + half];\n"
     "        xe = xe * scale;\n"
     "        xo = xo * scale;"),
    ("rope: no fma in rotation",
     "        re = fmaf(-xo, s[j], re); /* vfnmadd231ps: re - xo*sin, one rounding */",
     "        re = re - xo * s[j];"),
    ("rope: sin sign swapped",
     "        re = fmaf(-xo, s[j], re); /* vfnmadd231ps: re - xo*sin, one rounding */\n"
     "        ro = fmaf(xo, c[j], ro);  /* vfmadd231ps: ro + xo*cos, one rounding */",
     "        re = fmaf(xo, s[j], re);\n"
     "        ro = fmaf(-xo, c[j], ro);"),
    ("rope: pos 0 also rotates",
     "    if (pos == 0) {\n"
     "        /* %%rmsnorm_only",
     "    if (pos == -1) {\n"
     "        /* %%rmsnorm_only"),
    ("rope: fma other product",
     "        float re = xe * c[j];\n"
     "        float ro = xe * s[j];\n"
     "        re = fmaf(-xo, s[j], re);",
     "        float re = -xo * s[j];\n"
     "        float ro = xe * s[j];\n"
     "        re = fmaf(xe, c[j], re);"),
    ("quant: no floor",
     "        wmax = (wmax > Q_FLOOR) ? wmax : Q_FLOOR; /* vmaxss wmax, eps (:84) */",
     "        wmax = (wmax > 0.0f) ? wmax : 1e-30f;"),
    ("quant: NaN-free max",
     "    return (a > b) ? a : b;",
     "    return fmaxf(a, b);"),
    ("quant: vectors scanned in order",
     "            float lo = vmax(vmax(a[0], a[1]), vmax(a[2], a[3]));",
     "            float lo = vmax(vmax(vmax(a[0], a[1]), a[2]), a[3]);"),
    ("quant: lanes i+4 first",
     "        float p0 = vmax(m[0], m[4]), p1 = vmax(m[1], m[5]), p2 = vmax(m[2], m[6]), p3 = vmax(m[3], m[7]);",
     "        float p0 = vmax(m[4], m[0]), p1 = vmax(m[5], m[1]), p2 = vmax(m[6], m[2]), p3 = vmax(m[7], m[3]);"),
    ("fp env: DAZ without FTZ",
     "        _mm_setcsr(old | 0x8040u); /* FTZ (bit 15) + DAZ (bit 6) */",
     "        _mm_setcsr(old | 0x0040u);"),
    ("fp env: FTZ without DAZ",
     "        _mm_setcsr(old | 0x8040u); /* FTZ (bit 15) + DAZ (bit 6) */",
     "        _mm_setcsr(old | 0x8000u);"),
    ("quant: recip from wmax",
     "        float recip = 1.0f / scale;               /* vdivss (:88) */",
     "        float recip = 127.0f / wmax;"),
    ("quant: divide instead of recip",
     "            out_q[g * gs + i] = code_vec(x[i] * recip);",
     "            out_q[g * gs + i] = code_vec(x[i] / scale);"),
    ("quant: truncation",
     "        i = (int32_t)nearbyintf(v);",
     "        i = (int32_t)v;"),
    ("quant: allow -128",
     "    if (i < -127)\n"
     "        i = -127;\n"
     "    return (int8_t)i;",
     "    return (int8_t)i;"),
    ("quant: scale = wmax*(1/127)",
     "        float scale = wmax / 127.0f;              /* vdivss (:86) */",
     "        float scale = wmax * (1.0f / 127.0f);"),
    ("tail: round half away",
     "    return (int8_t)(int32_t)nearbyintf(v);",
     "    return (int8_t)(int32_t)roundf(v);"),
    ("emb: scale index per 32",
     "        out[i] = (float)q[i] * s[i >> 6];",
     "        out[i] = (float)q[i] * s[i >> 5];"),
    ("f16: truncate",
     "    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))\n"
     "        q += 1u; /* a carry into the exponent is the correct result, up to Inf */",
     "    (void)rem;"),
    ("f16: ties away",
     "    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))",
     "    if (rem >= 0x1000u)"),
    ("f16: flush subnormals",
     "        if (e < -10)\n"
     "            return (uint16_t)sign;",
     "        if (e < 1)\n"
     "            return (uint16_t)sign;"),
    ("rope_only: rotates at pos 0",
     "    if (pos == 0)\n"
     "        return;\n"
     "    const float *c = cos_table",
     "    const float *c = cos_table"),
    ("rope_only: no fma",
     "            re = fmaf(-up, s[j], re);",
     "            re = re - up * s[j];"),
    ("llama3: divides the high band",
     "        double ifl = (wavelen > low_wl) ? (double)((long double)inv / f) : inv;",
     "        double ifl = (wavelen < low_wl) ? (double)((long double)inv / f) : inv;"),
    ("llama3: interpolation weights swapped",
     "        double smoothed = (double)((1.0L - (long double)smooth) * ((long double)ifl / f) +\n"
     "                                   (long double)smooth * (long double)ifl);",
     "        double smoothed = (double)((long double)smooth * ((long double)ifl / f) +\n"
     "                                   (1.0L - (long double)smooth) * (long double)ifl);"),
    ("llama3: no medium band",
     "        int medium = wavelen >= high_wl && wavelen <= low_wl;",
     "        int medium = wavelen >= low_wl && wavelen <= high_wl;"),
    ("rmsnorm: (s*w)*x",
     "        float t = s * x[i];\n"
     "        o[i] = t * weight[i];",
     "        float t = s * weight[i];\n"
     "        o[i] = t * x[i];"),
]


def _run(name, a, b, orig, work):
    d = os.path.join(work, "".join(ch if ch.isalnum() else "_" for ch in name))
    os.makedirs(d)
    for f in ("v7_oracle_avx2.c", "v7_oracle.h", "v7_oracle_fpenv.h"):
        shutil.copy(os.path.join(ORACLE, f), d)
    with open(os.path.join(d, "v7_oracle.c"), "w") as fh:
        fh.write(orig.replace(a, b))
    so = os.path.join(d, "liboracle.so")
    subprocess.run(["gcc", "-O2", "-mfma", "-fPIC", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-shared", "-o", so,
                    os.path.join(d, "v7_oracle.c"), os.path.join(d, "v7_oracle_avx2.c"), "-lm", "-lpthread"],
                   check=True, capture_output=True)
    env = dict(os.environ, V7G_ORACLE_LIB=so)
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(ROOT, "tests", "test_oracle.py"), "-q", "-x",
                        "-k", "not avx2", "-p", "no:cacheprovider"], capture_output=True, text=True, cwd=ROOT,
                       env=env, timeout=600)
    return name, r.returncode


def test_every_planted_mistake_fails_a_pin():
    orig = open(os.path.join(ORACLE, "v7_oracle.c")).read()
    for name, a, _ in MUTANTS:
        assert orig.count(a) == 1, f"mutant {name!r}: its pattern no longer matches the oracle source once"
    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed to build the mutants")
    with tempfile.TemporaryDirectory() as work:
        workers = max(1, min(8, len(os.sched_getaffinity(0))))
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            results = list(pool.map(lambda m: _run(m[0], m[1], m[2], orig, work), MUTANTS))
    survivors = [n for n, rc in results if rc == 0]
    assert not survivors, f"planted mistakes not caught by any pin: {survivors}"
