#!/bin/sh
# expected_kl.txt: the output of the reference's own KL sanity check (tests/test_kl.c of the reference), compiled
# from its sources by oracle/Makefile (make -C oracle ref) and run on the CPU: 8 synthetic groups, 64 queries each,
# mean / max KL divergence and mean relative output error per body.
set -e
HERE=$(cd "$(dirname "$0")" && pwd)
make -C "$HERE/../../oracle" ref >/dev/null
"$HERE/../../oracle/_ref/test_kl" > "$HERE/expected_kl.txt"
