"""Copies the reference's external test corpus (data files only: the upstream
stas/tiny-random-llama-2 model at revision
3579d71fd57e04f5a364d824d3a2ec3e913dbb67, its config and the logits corpus
generated with transformers 4.53.2 on CPU torch, tests/reference_corpus/
MANIFEST.md:1-60) into this folder, checking each file's SHA-256 against the
reference manifest. Run once where /root/reference exists; the copies are
committed, so the tests never read the reference tree."""
import hashlib
import os
import shutil
import sys

SRC = "/root/reference/tests/reference_corpus"
HERE = os.path.dirname(os.path.abspath(__file__))
FILES = {  # MANIFEST.md:13-29
    "config.json": "9197475bfcc987a4f9361dbc22b33397b101372c137c228b6a6fd7e4adf21622",
    "model.safetensors": "852db1b39acb2336abc997440c6f6d6e4ab640f91e5e2aa9e2488d5794159d30",
    "corpus.json": "f4ade303b1b7b3264e86caa15b77cdb2805244e1142b9b74225ed3f36438f1d0",
}


def main():
    for name, digest in FILES.items():
        data = open(os.path.join(SRC, name), "rb").read()
        if hashlib.sha256(data).hexdigest() != digest:
            sys.exit(f"{name}: SHA-256 differs from the reference manifest")
        shutil.copyfile(os.path.join(SRC, name), os.path.join(HERE, name))
        print(name, len(data), digest)


if __name__ == "__main__":
    main()
