"""The reference's sampling draws (StdRng::seed_from_u64 + StandardUniform
f32, src/model.rs:629 and src/tensor.rs:1204): the oracle's restatement
against published vectors, and the library's own copy against the oracle.

rand 0.10.2 / rand_core 0.10.1 / chacha20 0.10.2 are not in the reference
tree.  The ChaCha block function is pinned by RFC 7539 (20 rounds) and, at
8 and 12 rounds, by the all-zero key and IV vectors of the ChaCha test-vector
draft (draft-strombergson-chacha-test-vectors-00, TC1, 256-bit key), so the
12-round block StdRng uses is pinned; the PCG XSH-RR output function by the
PCG reference demo; the crates' own steps (the seed expansion, StdRng's key
layout, counter, stream and word order, the f32 conversion) by the
value-stability vectors those crates' own tests hold."""
import numpy as np
import pytest

from oracle import oracle as O


def test_chacha_block_rfc7539():
    # RFC 7539 section 2.3.2: key 00..1f, nonce 00:00:00:09:00:00:00:4a:00:00:00:00,
    # block count 1 (words 12..15 = 1, 0x09000000, 0x4a000000, 0)
    key = np.array([int.from_bytes(bytes(range(4 * i, 4 * i + 4)), "little") for i in range(8)], np.uint32)
    out = O.chacha_block(key, (0x09000000 << 32) | 1, 0x4a000000, 20)
    assert [int(x) for x in out] == [
        0xe4e7f110, 0x15593bd1, 0x1fdd0f50, 0xc47120a3, 0xc7f4d1c7, 0x0368c033, 0x9aaa2204, 0x4e6cd4c3,
        0x466482d2, 0x09aa9f07, 0x05d7c214, 0xa2028bd9, 0xd19c12b5, 0xb94e16de, 0xe883d0cb, 0x4e3c50a2]
    # RFC 7539 appendix A.1, test vector 1: all-zero key, nonce and counter
    z = O.chacha_block(np.zeros(8, np.uint32), 0, 0, 20)
    assert b"".join(int(x).to_bytes(4, "little") for x in z).hex() == (
        "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
        "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586")


def test_chacha_8_and_12_round_blocks():
    # draft-strombergson-chacha-test-vectors-00, TC1 (all-zero 256-bit key and
    # 64-bit IV, block 0): ChaCha8 and ChaCha12 keystream (ChaCha20's is RFC
    # 7539 A.1 above)
    def ks(rounds):
        z = O.chacha_block(np.zeros(8, np.uint32), 0, 0, rounds)
        return b"".join(int(x).to_bytes(4, "little") for x in z).hex()
    assert ks(8) == ("3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
                     "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42")
    assert ks(12) == ("9bf49a6a0755f953811fce125f2683d50429c3bb49e074147e0089a52eae155f"
                      "0564f879d27ae3c02ce82834acfa8c793a629f2ca0de6919610be82f411326be")


def test_rand_crates_value_stability_vectors():
    """The known answers of the crates' own value-stability tests, through
    the oracle's functions."""
    M, INC, MASK = 6364136223846793005, 11634580027462260723, 2**64 - 1
    # rand_core, test_seed_from_u64: an 8-byte seed from seed_from_u64(0) reads
    # back as 5029875928683246316; StdRng's 32-byte seed starts with the same
    # two PCG32 outputs
    key0 = [int(x) for x in O.stdrng_key(0)]
    assert key0[0] | (key0[1] << 32) == 5029875928683246316
    # rand, rngs/std.rs test_stdrng_construction: StdRng::from_seed of this
    # seed gives next_u64 10719222850664546238; a second StdRng seeded from the
    # next 32 bytes of the first gives 14064965282130556830
    seed = bytes([1, 0, 0, 0, 23, 0, 0, 0, 200, 1, 0, 0, 210, 30, 0, 0] + [0] * 16)
    key = np.frombuffer(seed, "<u4").astype(np.uint32)
    w = [int(x) for x in O.chacha_block(key, 0, 0, 12)]
    assert w[0] | (w[1] << 32) == 10719222850664546238
    w2 = [int(x) for x in O.chacha_block(np.array(w[2:10], np.uint32), 0, 0, 12)]
    assert w2[0] | (w2[1] << 32) == 14064965282130556830
    # rand, distr/float.rs value_stability: StandardUniform f32 draws from the
    # tests' Pcg32::new(0x6f44f5646c2a7334, INC) source (increment (INC << 1) | 1,
    # the state stepped once after adding it, each output taken from the state
    # before its step)
    inc = ((INC << 1) | 1) & MASK
    st = ((0x6f44f5646c2a7334 + inc) * M + inc) & MASK
    draws = []
    for _ in range(3):
        draws.append(np.float32(O.uniform_f32(O.pcg_xsh_rr(st))))
        st = (st * M + inc) & MASK
    assert draws == [np.float32(0.0035963655), np.float32(0.7346052), np.float32(0.09778172)]
    # and the oracle's draws of seed 0 are the conversion of that stream's words
    u = O.stdrng_uniform(0, 2)
    b = O.chacha_block(np.array(key0, np.uint32), 0, 0, 12)
    assert [float(x) for x in u] == [O.uniform_f32(int(b[0])), O.uniform_f32(int(b[1]))]


def test_chacha_rounds_and_counter():
    key = O.stdrng_key(5)
    # fewer rounds give a different block; the counter and stream words move it
    assert not np.array_equal(O.chacha_block(key, 0, 0, 12), O.chacha_block(key, 0, 0, 20))
    assert not np.array_equal(O.chacha_block(key, 0, 0, 12), O.chacha_block(key, 1, 0, 12))
    assert not np.array_equal(O.chacha_block(key, 0, 0, 12), O.chacha_block(key, 0, 1, 12))


def test_pcg_output_function_demo_sequence():
    # pcg32 reference demo (srandom(42, 54)): output of the state before each
    # advance, increment (54 << 1) | 1
    M, MASK, inc = 6364136223846793005, 2**64 - 1, (54 << 1) | 1
    st = ((0 * M + inc) & MASK) + 42
    st = (st * M + inc) & MASK
    outs = []
    for _ in range(6):
        old, st = st, (st * M + inc) & MASK
        outs.append(O.pcg_xsh_rr(old))
    assert outs == [0xa15c02b7, 0x7b47f409, 0xba1d3330, 0x83d2f293, 0xbfa4784b, 0xcbed606e]


def test_stdrng_stream_structure():
    seed = 987654321
    key = O.stdrng_key(seed)
    # seed expansion: eight PCG32 outputs, the state advanced before each
    M, INC, MASK = 6364136223846793005, 11634580027462260723, 2**64 - 1
    st, exp = seed, []
    for _ in range(8):
        st = (st * M + INC) & MASK
        exp.append(O.pcg_xsh_rr(st))
    assert [int(x) for x in key] == exp
    # draws: the ChaCha12 words of blocks 0, 1, ... in order, top 24 bits
    u = O.stdrng_uniform(seed, 40)
    words = np.concatenate([O.chacha_block(key, b, 0, 12) for b in range(3)])[:40]
    assert np.array_equal(u, ((words >> 8).astype(np.float64) * 2.0**-24).astype(np.float32))
    assert u.min() >= 0.0 and u.max() < 1.0


def test_library_stdrng_matches_oracle():
    T = pytest.importorskip("tinyminigo_amd")
    for seed in (0, 1, 42, 2**64 - 1, 1234567890123):
        assert np.array_equal(T.stdrng_uniform(seed, 300), O.stdrng_uniform(seed, 300)), seed
    big = T.stdrng_uniform(42, 20000)
    assert abs(float(big.mean()) - 0.5) < 0.01
