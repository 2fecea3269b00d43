"""The committed profile summaries: each one states the rocprofv3 command
that produced it, and that command runs only files of this repository (the
bench, or a program built from committed sources), never a scratch script."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILES = os.path.join(ROOT, "profiles")
FILES = sorted(f for f in os.listdir(PROFILES) if not f.startswith("."))


def test_profiles_are_short_text():
    assert FILES, "no profile summaries"
    for f in FILES:
        assert f.endswith((".txt", ".md")), f
        assert os.path.getsize(os.path.join(PROFILES, f)) < 16 * 1024, f"{f} is not a short summary"


@pytest.mark.parametrize("name", FILES)
def test_profile_states_a_command_over_committed_files(name):
    text = open(os.path.join(PROFILES, name)).read()
    assert "rocprofv3" in text, f"{name}: no rocprofv3 command"
    assert "_work" not in text, f"{name}: cites scratch files"
    paths = re.findall(r"\$REPO/([\w./-]+)", text)
    assert paths, f"{name}: the command names no repository file"
    for p in paths:
        if p.startswith("gpurun_out/"):
            continue  # where the run writes its results
        src = os.path.join(ROOT, p)
        # a built program must have its source beside it
        assert os.path.exists(src) or os.path.exists(src + ".cpp"), f"{name}: {p} is not in the repository"
