"""`python -m inference_engine_rust_amd [-m MODEL] [-t TOKENIZER] [-n N] [--chat STYLE] PROMPT`:
the greedy text continuation command line of src/main.rs."""
import sys

from .frontend import main

sys.exit(main())
