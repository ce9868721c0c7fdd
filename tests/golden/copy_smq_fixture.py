"""Copies the reference's own .smq model file into tests/golden/ as a data fixture.

tools/CreateBenchmarkModel/benchmark-model.smq in the reference is a tiny GPT-2 style
TransformerModel (vocab 50, context 32, d 64, 2 layers, 4 heads) written by SmqWriter with
every parameter Q8_0-quantized at block 32 and named tensor_000 .. tensor_028 in parameter
order.  It is data (no code): the loader tests read it with the backend's parser and with the
checker's independent one.  Run in a container that has the reference:

    python tests/golden/copy_smq_fixture.py
"""
import hashlib
import os
import shutil

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/tools/CreateBenchmarkModel/benchmark-model.smq"
DST = os.path.join(HERE, "benchmark_model.smq")


def main():
    shutil.copyfile(SRC, DST)
    with open(DST, "rb") as f:
        print(DST, hashlib.sha256(f.read()).hexdigest())


if __name__ == "__main__":
    main()
