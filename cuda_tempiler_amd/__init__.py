"""cuda_tempiler_amd -- native side of the gfx950 (MI355X) plugin for the Tempolator pipeline.

  csrc/        the C-ABI shim and the FMHA translation unit (HIP)
  build.py     hipcc build of libtempo_gfx950.so (freezes skeletons into the shipped
               deliveries first)
  capi.py      ctypes binding of include/tempo_gfx950.h

The kernels themselves live in the plugin's skeletons (tempo/plugins/gfx950/skeletons) and
their frozen shipped copies (kernels/shipped/<op>/gfx950).
"""
