import pathlib
import sys

RACINE = pathlib.Path(__file__).resolve().parents[1]
for p in (str(RACINE), str(RACINE / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
