"""Bit-packed inference (silogic.bitpacking) on the MI355X HIP kernels.

Same public names and packed formats as the reference
(silogic/bitpacking/__init__.py:41-71): ``[dim, n_words]`` int64 for FC
activations and ``[dim, L, nw_B]`` for conv activations, 64 samples per
word, sample ``b`` at bit ``b % 64`` of word ``b // 64``; logits divided by
the GroupSum ``tau``. Every computation runs on the GPU; numpy inputs are
copied there and numpy results returned.

    from silogic_amd.bitpacking import convert_logic_net
    bp = convert_logic_net(trained_logic_net)
    logits = bp(x_uint8)               # [B, num_classes] float32
"""
from .. import _lib
from .convert import convert_conv_tree_layer, convert_head, convert_layer, convert_logic_conv_net, \
    convert_logic_net
from .ops import apply_gate, code_to_gate16, group_sum_packed, mask_last_word, n_words, pack_bits, \
    unpack_bits
from .packed_layer import (BitpackedConvLUTLayer, BitpackedConvTreeLayer, BitpackedFCLayer,
                           BitpackedGroupSumHead, BitpackedLUTLayer, pack_conv_input,
                           packed_or_pool, packed_unfold, unpack_conv_output)
from .packed_model import (BitpackedConvGPUNet, BitpackedConvNet, BitpackedNet, packed_or_pool_gpu,
                           packed_unfold_gpu)

# The reference exports HAS_TRITON (its GPU kernels available); here the GPU
# kernels are the HIP library's.
HAS_HIP = _lib.available()
HAS_TRITON = HAS_HIP

__all__ = [
    "convert_logic_net", "convert_logic_conv_net", "convert_layer", "convert_head",
    "convert_conv_tree_layer",
    "BitpackedNet", "BitpackedConvNet", "BitpackedConvGPUNet", "packed_unfold_gpu",
    "packed_or_pool_gpu", "pack_bits", "unpack_bits", "n_words", "group_sum_packed",
    "mask_last_word", "code_to_gate16", "apply_gate", "BitpackedFCLayer", "BitpackedLUTLayer",
    "BitpackedConvTreeLayer", "BitpackedConvLUTLayer", "BitpackedGroupSumHead",
    "pack_conv_input", "unpack_conv_output", "packed_unfold", "packed_or_pool",
    "HAS_HIP", "HAS_TRITON",
]
