"""Every citation of the reference in this repository's sources names a file that exists and a line
range inside it (path:line or path:first-last).  Runs where the reference tree is present."""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
PAT = re.compile(r"(?<![\w/])((?:src|tools|bench)/[\w./-]+\.(?:c|h|m|metal|py)|README\.md|COMPARISON\.md|Makefile)"
                 r":(\d+)(?:-(\d+))?")
SKIP_DIRS = {".git", "_work", "gpurun_out", "__pycache__", ".pytest_cache", "build", "_ref"}
TEXT = (".c", ".h", ".hip", ".py", ".md", ".S", ".json", "Makefile")
# review files written about this repository cite its own tree as well as the reference
NOT_SOURCES = {"VERDICT.md", "ADVICE.md", "SURVEY.md", "BASELINE.md"}


def sources():
    for root, dirs, files in os.walk(REPO):
        dirs[:] = [d for d in dirs if d not in SKIP_DIRS]
        for f in files:
            if f.endswith(TEXT) and f not in NOT_SOURCES:
                yield os.path.join(root, f)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="reference tree not present")
def test_reference_citations_in_range():
    lens, bad = {}, []
    for path in sources():
        with open(path, errors="ignore") as f:
            for i, line in enumerate(f, 1):
                for m in PAT.finditer(line):
                    p, a, b = m.group(1), int(m.group(2)), int(m.group(3) or m.group(2))
                    if p not in lens:
                        fp = os.path.join(REF, p)
                        lens[p] = sum(1 for _ in open(fp, errors="ignore")) if os.path.isfile(fp) else -1
                    n = lens[p]
                    if n < 0 or a < 1 or a > b or b > n:
                        bad.append(f"{os.path.relpath(path, REPO)}:{i}: {m.group(0)} ({p} has {n} lines)")
    assert not bad, "\n".join(bad)
