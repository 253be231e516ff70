"""Token ids <-> text, the reference's `tok` helper (tok/src/main.rs:1-23) on
the same library (Hugging Face tokenizers, here through its Python binding):

    python tok.py encode "prompt text"   -> space-separated ids (special tokens added, e.g. BOS)
    python tok.py decode 1 2 3 ...       -> text (special tokens kept)

The tokenizer file is ./models/tinyllama/tokenizer.json as in the reference,
or RFP4_TOKENIZER.  llama_run reads the ids (arguments or PROMPT_IDS) and
prints "output ids: ..." for `decode`.
"""
import os
import sys

DEFAULT_TOKENIZER = "./models/tinyllama/tokenizer.json"


def load(path=None):
    from tokenizers import Tokenizer

    return Tokenizer.from_file(path or os.environ.get("RFP4_TOKENIZER") or DEFAULT_TOKENIZER)


def encode(tk, text):
    return tk.encode(text, add_special_tokens=True).ids


def decode(tk, ids):
    return tk.decode(ids, skip_special_tokens=False)


def main(argv):
    if len(argv) < 2 or argv[1] not in ("encode", "decode"):
        print("usage: tok encode <text> | tok decode <id...>", file=sys.stderr)
        return 0  # the reference prints usage and exits normally
    tk = load()
    if argv[1] == "encode":
        print(" ".join(str(i) for i in encode(tk, " ".join(argv[2:]))))
    else:
        print(decode(tk, [int(s) for s in argv[2:]]))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
