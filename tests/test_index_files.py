"""Index files on the CPU: the byte layout the reference writes and reads
(build_index.cu:503-557, chimera_index.cu:79-164, ivf_pg.cpp:136-164,
io.cpp:94-108), the load-time failure contract with the reference's
exception types and messages (chimera_index.cu:27-36,58-61,82-105,146-155),
the centroid reader's search for the float32 [K, 128] dataset blob a cuVS
file carries (ivf_pg.cpp:67-74), and the candidate workspace's visit bound."""
import shutil
import struct

import numpy as np
import pytest

from chimera_amd import capi, synthetic

N_CLUSTERS, EX_BITS = 24, 3


@pytest.fixture(scope="module")
def saved(chimera_mod, tmp_path_factory):
    rng = np.random.default_rng(17)
    centres = synthetic.unit_centres(rng, 8, 128)
    lens = rng.integers(1, 12, size=60).astype(np.int32)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    d = tmp_path_factory.mktemp("ix")
    idx = chimera_mod._build_index(emb, lens.tolist(), N_CLUSTERS, EX_BITS, str(d))
    return d, idx


def fresh_copy(saved, tmp_path):
    d, _ = saved
    dst = tmp_path / "copy"
    shutil.copytree(d, dst)
    return dst


def test_file_sizes_and_byte_layout(saved):
    d, idx = saved
    n, k, w = int(idx["num_embeddings"]), N_CLUSTERS, 1 + EX_BITS
    m = idx["doc_lens"].size
    raw = (d / "doclens.bin").read_bytes()
    assert len(raw) == 4 + 4 * m
    assert struct.unpack_from("<i", raw)[0] == m
    assert np.array_equal(np.frombuffer(raw, "<i4", offset=4), idx["doc_lens"])

    raw = (d / "doc_1bit.bin").read_bytes()
    assert len(raw) == 40 + 64 + 16 * n + 4 * n + 4 * n
    assert struct.unpack_from("<5Q", raw) == (n, 128, k, EX_BITS, 128)
    assert np.array_equal(np.frombuffer(raw, np.uint8, 64, 40), idx["flips"])
    o = 104
    assert np.array_equal(np.frombuffer(raw, "<u8", 2 * n, o), idx["one_bit_codes"].reshape(-1))
    o += 16 * n
    assert np.array_equal(np.frombuffer(raw, "<f4", n, o), idx["one_bit_factors"])
    o += 4 * n
    assert np.array_equal(np.frombuffer(raw, "<f4", n, o), idx["full_bit_factors"])

    raw = (d / "doc_full.bin").read_bytes()
    assert len(raw) == n * 16 * w
    assert np.array_equal(np.frombuffer(raw, np.uint8), idx["full_bit_codes"].reshape(-1))

    raw = (d / "cluster_1bit.bin").read_bytes()
    assert len(raw) == n * 28
    codes = np.frombuffer(raw, np.uint8, 16 * n, 0).reshape(n, 16)
    f1 = np.frombuffer(raw, "<f4", n, 16 * n)
    docs = np.frombuffer(raw, "<i4", n, 20 * n)
    tok2pos = np.frombuffer(raw, "<u4", n, 24 * n)

    raw = (d / "ivf.bin").read_bytes()
    assert len(raw) == 8 + 4 * n + 8 * (k + 1)
    assert struct.unpack_from("<Q", raw)[0] == n
    inv = np.frombuffer(raw, "<u4", n, 8)
    cpos = np.frombuffer(raw, "<u8", k + 1, 8 + 4 * n)
    assert cpos[0] == 0 and cpos[-1] == n and np.all(np.diff(cpos.astype(np.int64)) >= 0)

    # the arrays agree with one another: position p of the cluster order
    # holds token inv[p]; tokens ascend within a cluster (ivf_pg.cpp:110-126)
    tok_codes = np.frombuffer(idx["one_bit_codes"].tobytes(), np.uint8).reshape(n, 16)
    assert np.array_equal(codes, tok_codes[inv])
    assert np.array_equal(f1, idx["one_bit_factors"][inv])
    token_doc = np.repeat(np.arange(m, dtype=np.int32), idx["doc_lens"])
    assert np.array_equal(docs, token_doc[inv])
    assert np.array_equal(tok2pos[inv], np.arange(n, dtype=np.uint32))
    for c in range(k):
        assert np.all(np.diff(inv[cpos[c]:cpos[c + 1]].astype(np.int64)) > 0)


def test_saved_index_reads_back(chimera_mod, saved):
    d, idx = saved
    back = chimera_mod._read_index(str(d))
    for key, v in idx.items():
        if isinstance(v, np.ndarray):
            assert np.array_equal(back[key], v), key
        else:
            assert back[key] == v, key


def header_patch(path, field, value):
    raw = bytearray(path.read_bytes())
    struct.pack_into("<Q", raw, 8 * field, value)
    path.write_bytes(bytes(raw))


@pytest.mark.parametrize("field,value", [(0, 0), (0, 1 << 31), (1, 63), (1, 129), (2, 0), (2, 10 ** 6), (3, 0),
                                         (3, 8)], ids=["n0", "n-int-max", "d63", "d129", "k0", "k>n", "ex0", "ex8"])
def test_corrupt_header_is_rejected(chimera_mod, saved, tmp_path, field, value):
    d = fresh_copy(saved, tmp_path)
    header_patch(d / "doc_1bit.bin", field, value)
    with pytest.raises(RuntimeError, match="^Invalid Chimera index header: .*doc_1bit.bin$"):
        chimera_mod._read_index(str(d))


def test_padded_dimension_mismatch(chimera_mod, saved, tmp_path):
    d = fresh_copy(saved, tmp_path)
    header_patch(d / "doc_1bit.bin", 4, 64)
    with pytest.raises(RuntimeError, match="^Index file padded_dim=64 does not match compiled PADDED_DIM=128"):
        chimera_mod._read_index(str(d))


@pytest.mark.parametrize("name,keep,message", [
    ("doc_1bit.bin", 40 + 10, "Failed to read rotator from"),
    ("doc_1bit.bin", 40 + 64 + 100, "Failed to read quantized payload from"),
    ("doc_full.bin", 7, "Failed to read full-code payload from"),
    ("cluster_1bit.bin", 28 * 3, "Invalid clustered index payload: "),
    ("ivf.bin", 12, "Failed to read IVF lists from"),
    ("doclens.bin", 2, "Failed to read input file: "),
])
def test_truncated_files_are_rejected(chimera_mod, saved, tmp_path, name, keep, message):
    d = fresh_copy(saved, tmp_path)
    p = d / name
    p.write_bytes(p.read_bytes()[:keep])
    with pytest.raises(RuntimeError, match="^" + message):
        chimera_mod._read_index(str(d))


def test_clustered_payload_must_have_the_exact_size(chimera_mod, saved, tmp_path):
    d = fresh_copy(saved, tmp_path)
    p = d / "cluster_1bit.bin"
    p.write_bytes(p.read_bytes() + b"\0")  # one byte too many (chimera_index.cu:146-155)
    with pytest.raises(RuntimeError, match="^Invalid clustered index payload: "):
        chimera_mod._read_index(str(d))


def test_missing_directory(chimera_mod, tmp_path):
    with pytest.raises(RuntimeError, match="^Chimera index directory does not exist: "):
        chimera_mod.ChimeraIndex.load(str(tmp_path / "absent"))


def test_option_errors_on_load(chimera_mod, saved, tmp_path):
    d, _ = saved
    # checked before any device is touched, in the reference's order
    with pytest.raises(ValueError, match="^nprobe must not exceed the number of clusters$"):
        chimera_mod.ChimeraIndex.load(str(d), nprobe=N_CLUSTERS + 1, k_refine=50, k_full_bit=10)
    with pytest.raises(ValueError, match="^k_full_bit must not exceed k_refine$"):
        chimera_mod.ChimeraIndex.load(str(d), nprobe=4, k_refine=10, k_full_bit=20)
    with pytest.raises(ValueError, match="^All Chimera search options must be positive$"):
        chimera_mod.ChimeraIndex.load(str(d), nprobe=0)
    # the nprobe check comes right after the header, before the other files
    bad = fresh_copy(saved, tmp_path)
    (bad / "doc_full.bin").write_bytes(b"")
    with pytest.raises(ValueError, match="^nprobe must not exceed"):
        chimera_mod.ChimeraIndex.load(str(bad), nprobe=N_CLUSTERS + 1, k_refine=50, k_full_bit=10)


def npy_blob(arr, version=1, descr=None):
    descr = descr or arr.dtype.descr[0][1]
    h = "{'descr': '%s', 'fortran_order': False, 'shape': (%s), }" % (
        descr, ", ".join(str(s) for s in arr.shape) + ("," if arr.ndim == 1 else ""))
    if version == 1:
        pad = (64 - (10 + len(h) + 1) % 64) % 64
        h = h + " " * pad + "\n"
        return b"\x93NUMPY\x01\x00" + struct.pack("<H", len(h)) + h.encode() + arr.tobytes()
    pad = (64 - (12 + len(h) + 1) % 64) % 64
    h = h + " " * pad + "\n"
    return b"\x93NUMPY\x02\x00" + struct.pack("<I", len(h)) + h.encode() + arr.tobytes()


@pytest.mark.parametrize("version", [1, 2])
def test_centroids_found_inside_a_graph_serialisation(chimera_mod, saved, tmp_path, version):
    """A file shaped like cuVS's: leading non-array bytes, a graph blob
    (uint32 [K, 32]), a decoy float32 array of another shape, then the
    float32 [K, 128] dataset. The reader must return that dataset."""
    d = fresh_copy(saved, tmp_path)
    _, idx = saved
    cents = idx["rotated_centroids"].reshape(N_CLUSTERS, 128)
    rng = np.random.default_rng(0)
    graph = rng.integers(0, N_CLUSTERS, (N_CLUSTERS, 32)).astype(np.uint32)
    decoy = rng.standard_normal((N_CLUSTERS, 64)).astype(np.float32)
    blob = (b"\x01\x00\x00\x00cagra-v4\x93garbage" + npy_blob(graph, version) + b"\x93NUMPYxx"
            + npy_blob(decoy, version) + struct.pack("<Q", 128) + npy_blob(cents, version) + b"\0" * 5)
    (d / "centroids.carga").write_bytes(blob)
    back = chimera_mod._read_index(str(d))
    assert np.array_equal(back["rotated_centroids"].reshape(N_CLUSTERS, 128), cents)


def test_centroid_file_without_the_dataset(chimera_mod, saved, tmp_path):
    d = fresh_copy(saved, tmp_path)
    wrong = np.zeros((N_CLUSTERS, 128), np.float64)  # float64 is not the dataset's type
    (d / "centroids.carga").write_bytes(b"junk" + npy_blob(wrong))
    with pytest.raises(RuntimeError, match=r"^No float32 \[24, 128\] centroid array found in "):
        chimera_mod._read_index(str(d))


def test_visit_bound():
    cpos = np.array([0, 5, 5, 12, 13, 40], np.uint64)  # sizes 5, 0, 7, 1, 27
    assert capi.visit_bound(cpos, 1) == 32 * 27
    assert capi.visit_bound(cpos, 2) == 32 * (27 + 7)
    assert capi.visit_bound(cpos, 9) == 32 * 40
    # the largest clusters' tokens times 32 must fit the 32-bit visit offsets
    big = np.array([0, 1 << 25, 1 << 26, (1 << 26) + 1], np.uint64)
    assert capi.visit_bound(big, 1) == 32 << 25
    with pytest.raises(capi.ChimeraError, match="32-bit") as e:
        capi.visit_bound(big, 2)
    assert e.value.code == capi.ERR_CAPACITY
    with pytest.raises(capi.ChimeraError, match="Invalid IVF cluster offsets"):
        capi.visit_bound(np.array([0, 5, 3], np.uint64), 1)
