"""Module-level switches of the hot path (core/global_env_config.py:99-109).

``use_layernorm`` gates ``norm1`` and ``use_shift_size_0`` forces W-MSA in
every block, as in the reference.  The reference's ``use_attn_mask`` /
``use_relative_position_bias`` / ``USE_FLASH_ATTENTION`` defaults are the
truthy string 'no use now'; here the corresponding constructor defaults are
plain ``True`` / ``True`` / ``False`` with the same effect on this path.
"""
use_layernorm = True
use_MLP = True
use_shift_size_0 = False
