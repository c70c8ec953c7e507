"""Host-side surface without a GPU (the reference's tests/cpp/test_tensor_cpu.cpp tier):
zero-copy Tensor views of CPU memory and their DLPack export, the Request / Response
setters, and the exception hierarchy of the pybind module."""
import pytest
import torch

import edge_fm


@pytest.mark.parametrize("dtype,edt", [(torch.bfloat16, edge_fm.DType.BFloat16), (torch.float32, edge_fm.DType.Float32),
                                       (torch.int32, edge_fm.DType.Int32), (torch.uint8, edge_fm.DType.UInt8)])
def test_cpu_tensor_view_dlpack_roundtrip(dtype, edt):
    src = (torch.arange(24) * 3).reshape(2, 3, 4).to(dtype)
    t = edge_fm.Tensor(src.data_ptr(), [2, 3, 4], edt, edge_fm.Device.CPU, 0)
    assert t.shape() == [2, 3, 4] and t.dtype() == edt and not t.empty()
    assert t.nbytes() == src.numel() * src.element_size() and t.data_ptr() == src.data_ptr()
    back = torch.from_dlpack(t.to_dlpack())
    assert back.dtype == dtype and back.shape == src.shape and back.data_ptr() == src.data_ptr()
    assert torch.equal(back, src)
    src[0, 0, 0] = 7   # a view, not a copy
    assert back[0, 0, 0].item() == 7


def test_tensor_views_are_not_owners():
    with pytest.raises(edge_fm.InvalidArgumentError):
        edge_fm.Tensor(0, [1], edge_fm.DType.Float32, edge_fm.Device.CPU, 0, True)
    assert edge_fm.Tensor().empty()


def test_request_surface():
    r = edge_fm.Request(3, [5, 6, 7])
    assert r.request_id() == 3 and r.token_ids() == [5, 6, 7]
    assert not r.has_embedding() and not r.has_position_ids() and not r.has_mrope_last_pos()
    r.set_stop_token_ids([9, 10])
    r.set_ignore_stop_tokens(True)
    assert r.stop_token_ids() == [9, 10] and r.ignore_stop_tokens()
    emb = torch.zeros(2, 8, dtype=torch.bfloat16)
    pos = torch.zeros(3, 3, dtype=torch.int32)
    te = edge_fm.Tensor(emb.data_ptr(), [2, 8], edge_fm.DType.BFloat16, edge_fm.Device.CPU, 0)
    tp = edge_fm.Tensor(pos.data_ptr(), [3, 3], edge_fm.DType.Int32, edge_fm.Device.CPU, 0)
    r2 = edge_fm.Request(0, [1, 100, 101], te, 100, tp, [4, 4, 4])
    assert r2.has_embedding() and r2.embed_token_id() == 100 and r2.has_position_ids()
    assert r2.mrope_last_pos() == [4, 4, 4] and r2.embedding().shape() == [2, 8]


def test_exception_hierarchy():
    for name in ("InvalidRequestError", "DeviceError", "ConfigurationError", "ModelNotLoadedError",
                 "OutOfMemoryError", "InternalError", "InvalidArgumentError"):
        assert issubclass(getattr(edge_fm, name), edge_fm.Error)
    assert issubclass(edge_fm.Error, RuntimeError)


def test_engine_config_errors_are_configuration_errors(tmp_path):
    # a compact-vocab view of a config whose model directory is missing
    cfg = tmp_path / "engine.json"
    cfg.write_text('{"prefill_model_path": "%s"}' % (tmp_path / "absent"))
    with pytest.raises(edge_fm.ConfigurationError):
        edge_fm.CompactVocab(str(cfg))
    cfg.write_text("{not json")
    with pytest.raises(edge_fm.ConfigurationError):
        edge_fm.CompactVocab(str(cfg))
