"""Library calls from several host threads on separate HIP streams, in a fresh
process so that their one-time per-kernel set-up also runs concurrently."""
if __name__ == "__main__":  # `python tests/<file>.py`, as the reference runs its tests
    import sys as _sys

    import pytest as _pytest
    _sys.exit(_pytest.main([__file__, "-q"]))
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

SCRIPT = Path(__file__).resolve().parent / "gpu_scripts" / "concurrent_streams.py"


def test_threads_on_separate_streams():
    print("[case] concurrent streams (subprocess)", flush=True)
    r = subprocess.run([sys.executable, str(SCRIPT)], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    assert r.stdout.strip().endswith("ok")
