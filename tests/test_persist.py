"""Prompt-cache files: format checks that need no GPU."""
import numpy as np
import pytest
import torch


def test_rejects_foreign_safetensors(tmp_path):
    from safetensors.torch import save_file

    from chronoquant_mlx_amd import load_prompt_cache
    f = str(tmp_path / "other.safetensors")
    save_file({"0.0": torch.zeros(2)}, f, metadata={"format": "something-else"})
    with pytest.raises(ValueError):
        load_prompt_cache(f, device="cpu")


def test_save_rejects_unknown_cache_type(tmp_path):
    from chronoquant_mlx_amd import save_prompt_cache

    class Foreign:
        state = []
        meta_state = ""
    with pytest.raises(TypeError):
        save_prompt_cache(str(tmp_path / "x.safetensors"), [Foreign()])


def _codes(rng, shape, bits):
    half = 1 << (bits - 1)
    return rng.integers(-half, half, size=shape).astype(np.int8)  # the codec's clip range


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("D", [128, 64, 12, 5])
def test_dense_pack_round_trip_and_bit_order(bits, D):
    # INT4 lanes from the oracle's packer -> dense stream -> INT4 lanes again,
    # bit-exact; each stream field read back one bit at a time is the code's
    # offset value (field d at stream bits [bits*d, bits*d + bits), LSB first)
    from chronoquant_mlx_amd.persist import dense_pack, dense_unpack
    from oracle.np_oracle import pack_int4_codes
    rng = np.random.default_rng(D * 10 + bits)
    codes = _codes(rng, (3, 2, 7, D), bits)
    codes[0, 0, 0] = -(1 << (bits - 1))           # both ends of the range
    codes[0, 0, 1] = (1 << (bits - 1)) - 1
    words = torch.from_numpy(pack_int4_codes(codes).view(np.int32)).view(torch.uint32)
    stream = dense_pack(words, D, bits)
    assert stream.dtype == torch.uint8 and stream.shape == (3, 2, 7, (D * bits + 7) // 8)
    s = stream.numpy()
    for idx in [(0, 0, 0), (0, 0, 1), (2, 1, 6), (1, 0, 3)]:
        for d in range(D):
            f = sum(((int(s[idx][(bits * d + i) // 8]) >> ((bits * d + i) % 8)) & 1) << i
                    for i in range(bits))
            assert f == int(codes[idx][d]) + (1 << (bits - 1)), (idx, d)
    back = dense_unpack(stream, D, bits)
    assert back.dtype == torch.uint32
    assert np.array_equal(back.view(torch.int32).numpy(), words.view(torch.int32).numpy())


def test_dense_pack_rejects_out_of_range_codes():
    from chronoquant_mlx_amd.persist import dense_pack, dense_unpack
    from oracle.np_oracle import pack_int4_codes
    codes = np.zeros((2, 16), np.int8)
    codes[1, 3] = 4                                   # does not fit 3 bits
    words = torch.from_numpy(pack_int4_codes(codes).view(np.int32)).view(torch.uint32)
    with pytest.raises(ValueError):
        dense_pack(words, 16, 3)
    with pytest.raises(ValueError):
        dense_pack(words, 16, 4)
    with pytest.raises(ValueError):
        dense_unpack(torch.zeros(2, 5, dtype=torch.uint8), 16, 3)   # 6 bytes expected


def test_dense_pack_chunking_is_seamless(monkeypatch):
    # rows are packed in chunks; a chunk size that does not divide the row
    # count gives the same stream as one chunk
    import chronoquant_mlx_amd.persist as persist
    from oracle.np_oracle import pack_int4_codes
    codes = _codes(np.random.default_rng(11), (4, 3, 9, 128), 3)
    words = torch.from_numpy(pack_int4_codes(codes).view(np.int32)).view(torch.uint32)
    whole = persist.dense_pack(words, 128, 3)
    monkeypatch.setattr(persist, "_CHUNK_ROWS", 5)
    assert torch.equal(persist.dense_pack(words, 128, 3), whole)
    back = persist.dense_unpack(whole, 128, 3)
    assert torch.equal(back.view(torch.int32), words.view(torch.int32))
