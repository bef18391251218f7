"""CPU checks of aether_load on crafted GGUF headers (no GPU needed): sizes that
would wrap 64-bit products, dimensions past int32, and non-positive config
values are refused by the reader before any device work, with the reason in
the last error (gguf.rs:297-397 reads such files; model_loader.rs:159-300
builds the config)."""
import numpy as np
import pytest

import aether_amd as A
from tests.gguf_writer import F32 as VF32
from tests.gguf_writer import I32, STR, U32, write_gguf

GOOD_META = [("general.architecture", STR, "llama"), ("llama.embedding_length", U32, 256),
             ("llama.block_count", U32, 1), ("llama.attention.head_count", U32, 2),
             ("llama.feed_forward_length", U32, 512), ("llama.rope.freq_base", VF32, 10000.0)]


def emb(vocab=512, d=256):
    return ("token_embd.weight", [d, vocab], 0, np.zeros(d * vocab * 4, np.uint8))


def load(tmp_path, meta, tensors):
    p = str(tmp_path / "crafted.gguf")
    write_gguf(p, meta, tensors)
    m = A.lib().aether_load(p.encode())
    return m, A.last_error()


@pytest.mark.parametrize("shape", [[256, 2 ** 60 + 32], [2 ** 31, 2], [2 ** 31 - 1, 2 ** 31 - 1, 2 ** 31 - 1]])
def test_shape_products_that_wrap_are_refused(tmp_path, shape):
    """A Q4_K tensor of [256, 2^60 + 32] has 2^68 + 8192 elements: the product
    wraps to 8192 in 64 bits and would pass the bounds check; each dimension
    past int32, or a product past 64 bits, is refused instead."""
    t = ("blk.0.attn_q.weight", shape, 12, np.zeros(4608, np.uint8))
    m, err = load(tmp_path, GOOD_META, [emb(), t])
    assert m is None
    assert "overflows" in err, err


def test_byte_size_that_wraps_is_refused(tmp_path):
    # (2^31-1)² × 2 F32 elements: the element count fits 64 bits, ×4 bytes does not
    t = ("blk.0.attn_q.weight", [2 ** 31 - 1, 2 ** 31 - 1, 2], 0, np.zeros(64, np.uint8))
    m, err = load(tmp_path, GOOD_META, [emb(), t])
    assert m is None and "overflows" in err, err


def test_tensor_past_the_end_is_refused(tmp_path):
    t = ("blk.0.attn_q.weight", [4096, 4096], 12, np.zeros(144, np.uint8))
    m, err = load(tmp_path, GOOD_META, [emb(), t])
    assert m is None and "out of bounds" in err, err


@pytest.mark.parametrize("key,value", [("llama.block_count", -1), ("llama.embedding_length", 0),
                                       ("llama.attention.head_count", -4), ("llama.feed_forward_length", -512),
                                       ("llama.embedding_length", 2 ** 31 - 1 + 1)])
def test_non_positive_or_huge_config_is_refused(tmp_path, key, value):
    meta = [(k, t, v) for k, t, v in GOOD_META if k != key]
    meta.append((key, I32, value) if -2 ** 31 <= value < 2 ** 31 else (key, U32, value))
    m, err = load(tmp_path, meta, [emb()])
    assert m is None
    assert "GGUF config" in err or "not a multiple" in err, err


def test_truncated_header_is_refused(tmp_path):
    p = tmp_path / "short.gguf"
    write_gguf(str(p), GOOD_META, [emb()])
    data = p.read_bytes()
    p.write_bytes(data[:60])
    assert A.lib().aether_load(str(p).encode()) is None
    assert "truncated" in A.last_error() or "bad value" in A.last_error(), A.last_error()
