"""Failure handling on the GPU: qh_fault_alloc forces each of qh_decoder_create's device allocations to fail in turn.
Every forced failure must come back as QH_ERR_NOMEM with nothing leaked, and the decoder built once the hook lets
every allocation through must decode exactly like one built without it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_decoder_create_survives_each_allocation_failure(qh, gpu):
    import torch
    import quanta_cpp_amd.qnt as qnt
    hp = qnt.HParams(vocab_size=4096, n_layers=2)
    tensors = qnt.synthetic_q4mix(77, hp)
    L = qh.lib()
    ref = qh.Decoder(hp, tensors, ctx_len=64)
    ids = np.random.default_rng(3).integers(0, hp.vocab_size, 9).astype(np.int32)
    ref.prefill(ids, 0, top_k=1)
    want = np.array(ref.hidden(), copy=True)
    ref.close()
    del ref
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free0 = torch.cuda.mem_get_info()[0]
    k = 0
    try:
        while True:
            L.qh_fault_alloc(k)
            try:
                dec = qh.Decoder(hp, tensors, ctx_len=64)
            except qh.QHError as e:
                assert f"status {qh.ERR_NOMEM}:" in str(e), str(e)
                k += 1
                assert k < 200
                continue
            break
    finally:
        L.qh_fault_alloc(-1)
    print(f"decoder created after {k} forced failures", flush=True)
    assert k >= 10  # the decoder makes that many device allocations at least
    dec.prefill(ids, 0, top_k=1)
    assert dec.hidden().tobytes() == want.tobytes()
    dec.close()
    del dec
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    # every allocation a failed create made was freed (a margin of a few MiB for the allocator's own bookkeeping)
    assert free0 - torch.cuda.mem_get_info()[0] < 8 << 20
