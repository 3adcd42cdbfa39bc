"""Helpers shared by the decoder tests: the synthetic-model module and the oracle decoder over a tensor set."""
from conftest import load_package


def qnt_module():
    load_package()
    import quanta_cpp_amd.qnt as qnt
    return qnt


def oracle_decoder(oracle, hp, tensors, ctx_len=None):
    return oracle.decoder_for(hp, tensors, ctx_len)
