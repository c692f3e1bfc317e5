"""Copies the one gob file the reference holds into this directory as a test
fixture (data only): examples/portuguese_gpt/portuguese_gpt.bin, which its
main.go:332-339 wrote with gob.NewEncoder(f).Encode(model.Params()) — a Go
process's []float32 as its first gob value (15103 parameters).

    python tests/golden/gob/copy_fixture.py [/root/reference]
"""
import os
import shutil
import sys

ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
src = os.path.join(ref, "examples", "portuguese_gpt", "portuguese_gpt.bin")
dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "portuguese_gpt_params.gob")
shutil.copyfile(src, dst)
print(dst, os.path.getsize(dst))
