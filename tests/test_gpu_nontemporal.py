"""The nontemporal (streaming-hint) kernel variants against the oracle.

Kernels switch to nontemporal loads / stores of their dense matrix from a
size threshold on (192 MiB by default), so the oracle-sized parity tests run
the plain variants.  Here the threshold is set to 0 for the duration of each
test (bs_nontemporal_min_bytes), so the same bit-exact checks run through the
streaming variants: fused compress (bf16, quantizing, fp8 inputs, packed),
decompress (raw, ReLU^2 with scale, packed, row batches), both gradient
kernels, amax and quantize."""
import pytest

from tests import test_gpu_codec as C
from tests import test_gpu_packed as P

pytestmark = pytest.mark.gpu

CASES = {
    "compress_bf16_129x131_s50": (C.test_compress_standalone_bf16, dict(shape=(129, 131), sparsity=0.5)),
    "compress_bf16_512x384_s90": (C.test_compress_standalone_bf16, dict(shape=(512, 384), sparsity=0.9)),
    "compress_special_values": (C.test_compress_special_values, dict(shape=(129, 131))),
    "compress_e4m3fn_input": (C.test_compress_fp8_inputs,
                              dict(dt=C.torch.float8_e4m3fn, code=C.O.E4M3FN, shape=(512, 384))),
    "shared_buffer": (C.test_shared_buffer_decompress_after_all_writes, {}),
    "overflow_contained": (C.test_buffer_overflow_is_flagged_and_contained, {}),
    "c1_round_trip": (C.test_c1_round_trip_bit_exact, {}),
    "unpack_row_batches": (C.test_unpack_row_batches, dict(shape=(448, 512))),
    "relu_grad": (C.test_relu_grad, {}),
    "relu2_grad_bf16": (C.test_relu2_grad_bf16, dict(shape=(256, 512))),
    "relu2_grad_fp8_scaled": (C.test_relu2_grad_and_square_fp8_scaled, dict(shape=(256, 512))),
    "relu2_every_bit_pattern": (C.test_relu2_paths_every_bit_pattern, {}),
    "to_fp8": (C.test_to_fp8, dict(shape=(1000, 4096))),
    "quantize_and_compress": (C.test_quantize_and_compress, dict(shape=(512, 1024))),
    "packed_standalone_bf16": (P.test_compress_packed_standalone, dict(shape=(320, 1024), code=C.O.BF16)),
    "packed_standalone_e4m3fn": (P.test_compress_packed_standalone, dict(shape=(129, 131), code=C.O.E4M3FN)),
    "packed_tensorbuffer_sequence": (P.test_compress_packed_tensorbuffer_sequence, {}),
    "packed_relu2_equal_raw": (P.test_relu2_unpack_and_grad_packed_equal_raw, {}),
}


@pytest.fixture
def nontemporal_everywhere(dev):
    from bitsparse_amd import _lib
    L = _lib.load()
    prev = L.bs_nontemporal_min_bytes(0)
    yield
    L.bs_nontemporal_min_bytes(prev)


@pytest.mark.parametrize("case", sorted(CASES))
def test_streaming_variant_matches_oracle(dev, nontemporal_everywhere, case):
    fn, kw = CASES[case]
    fn(dev, **kw)

