#!/bin/sh
# ChaCha20 keystream vectors from OpenSSL's RFC 7539 cipher (IV = 32-bit block
# counter || 96-bit nonce; with a zero nonce and counter < 2^32 this is the
# same block sequence as a 64-bit counter and zero stream id).  Writes one line
# per vector: KEYHEX COUNTER NBLOCKS then the keystream as 32-bit little-endian words.
# Usage: sh tests/golden/make_chacha20_vectors.sh > tests/golden/chacha20_keystream.txt
set -e
for spec in "000102030405060708090a0b0c0d0e0f101112131415161718191a1b1c1d1e1f 0 4" \
            "0000000000000000000000000000000000000000000000000000000000000000 0 2" \
            "c0ffee00deadbeef0123456789abcdeffedcba98765432100f1e2d3c4b5a6978 7 3"; do
    set -- $spec
    key=$1; ctr=$2; n=$3
    iv=$(printf '%08x' "$ctr" | sed 's/\(..\)\(..\)\(..\)\(..\)/\4\3\2\1/')000000000000000000000000
    words=$(head -c $((64 * n)) /dev/zero | openssl enc -chacha20 -K "$key" -iv "$iv" | od -An -tx4 -v | tr -s ' \n' ' ')
    echo "$key $ctr $n$words"
done
