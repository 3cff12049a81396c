#!/bin/sh
# Builds the reference's myl7/fss v0.7.1 DCF (vendored in the reference tree
# at third_party/myl7_fss, source files used unmodified and in place) into
# oracle/_ref/, one library per output group, plus oracle/ref_shim.cpp, and
# the gate-table dump driver oracle/ref_tables.cpp over the reference's
# header-only table builders, oracle/ref_suf_eval.cpp over its header-only
# eval_suf_ref, and oracle/ref_tape.cpp over its header-only TapeWriter.
# Compile definitions follow the reference's myl7_core target
# (CMakeLists.txt:84-93): kBlocks=8, kLambda=16, OpenSSL libcrypto, OpenMP.
# Outputs go only to oracle/_ref/ (git-ignored).  Without the reference tree
# this script does nothing and exits 0.
set -eu
HERE=$(cd "$(dirname "$0")" && pwd)
REF=${SUF_REFERENCE_ROOT:-/root/reference}
M="$REF/third_party/myl7_fss"
if [ ! -f "$M/src/dcf.c" ]; then
  echo "build_ref: reference tree not found at $REF; nothing built"
  exit 0
fi
OUT="$HERE/_ref"
mkdir -p "$OUT/obj"
CFLAGS="-O2 -fPIC -fopenmp -DkBlocks=8 -DkLambda=16 -I$M/include"
gcc $CFLAGS -c "$M/src/dcf.c" -o "$OUT/obj/dcf.o"
gcc $CFLAGS -c "$M/src/prg/aes128_mmo.c" -o "$OUT/obj/aes128_mmo.o"
g++ -std=c++17 -fno-gnu-unique $CFLAGS -I"$REF/include" -c "$HERE/ref_shim.cpp" -o "$OUT/obj/ref_shim.o"
for grp in bytes u128_le; do
  gcc $CFLAGS -c "$M/src/group/$grp.c" -o "$OUT/obj/group_$grp.o"
  g++ -shared -fopenmp -Wl,-Bsymbolic -o "$OUT/libmyl7ref_$grp.so.tmp" "$OUT/obj/dcf.o" "$OUT/obj/aes128_mmo.o" \
    "$OUT/obj/group_$grp.o" "$OUT/obj/ref_shim.o" -lcrypto
  mv "$OUT/libmyl7ref_$grp.so.tmp" "$OUT/libmyl7ref_$grp.so"
done
# The gate-table dump driver (tests/golden/make_tables.py runs it): the
# reference's header-only table and SUF builders, included in place.
g++ -std=c++17 -O1 -I"$REF/include" "$HERE/ref_tables.cpp" -o "$OUT/ref_tables.tmp"
mv "$OUT/ref_tables.tmp" "$OUT/ref_tables"
# The SUF reference-evaluation driver (tests/golden/make_suf_ref.py runs it).
g++ -std=c++17 -O1 -I"$REF/include" "$HERE/ref_suf_eval.cpp" -o "$OUT/ref_suf_eval.tmp"
mv "$OUT/ref_suf_eval.tmp" "$OUT/ref_suf_eval"
# The tape-record driver (tests/golden/make_tape.py runs it).
g++ -std=c++20 -O1 -I"$REF/include" "$HERE/ref_tape.cpp" -o "$OUT/ref_tape.tmp"
mv "$OUT/ref_tape.tmp" "$OUT/ref_tape"
echo "build_ref: built $OUT/libmyl7ref_bytes.so $OUT/libmyl7ref_u128_le.so $OUT/ref_tables $OUT/ref_suf_eval $OUT/ref_tape"
