"""MI355X-native (gfx950) quantized GEMM family with DSL_Tool's dispatcher API.

* ``dsl_tool_amd.gemm``       -- ``fp8_gemm``, ``fp4_gemm``, ``grouped_gemm``
  (the callables registered as ``gemm.*`` under backend ``hip``) and their
  packed-operand forms;
* ``dsl_tool_amd.quant``      -- GPU quantize/pack (E4M3, MXFP4, NVFP4);
* ``dsl_tool_amd.dispatcher`` -- registry / KernelDispatcher / REST / CLI;
* ``dsl_tool_amd.build``      -- hipcc build of ``_lib/libdsl_gemm.so``.
"""
__version__ = "0.1.0"
