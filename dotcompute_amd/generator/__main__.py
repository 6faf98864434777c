"""python -m dotcompute_amd.generator OUT_DIR FILE.cs [FILE.cs ...]"""
import sys

from . import generate

if __name__ == "__main__":
    if len(sys.argv) < 3:
        sys.exit(__doc__)
    for r in generate(sys.argv[2:], sys.argv[1]):
        km = r["km"]
        print(f"{km.full_name}: " + (f"HIP entry {r['entry']} ({r['dims']}-D)" if r["entry"] else f"CPU only: {r['error']}"))
