"""``python -m tribench_amd``: the harness command line."""
from .harness.cli import main

main()
