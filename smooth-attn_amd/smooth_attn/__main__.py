"""``python -m smooth_attn``: the benchmark command line (reference console
script ``smooth-attn``, pyproject.toml:36-37)."""
from .cli import main

if __name__ == "__main__":
    main()
