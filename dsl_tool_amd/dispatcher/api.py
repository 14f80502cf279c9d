"""FastAPI service over the dispatcher (endpoints of the reference's
dispatcher/api.py:48-108):

* ``GET  /health``
* ``GET  /api/v1/kernels``
* ``GET  /api/v1/kernels/{kernel_name}?backend=hip``
* ``POST /api/v1/kernels/run``  -> 404 ``kernel_not_found`` for an unknown
  name/backend, 400 ``kernel_dispatch_failed`` for any kernel error.

Run: ``uvicorn dsl_tool_amd.dispatcher.api:app --host 127.0.0.1 --port 8000``
"""
from __future__ import annotations

import logging
from contextlib import asynccontextmanager
from typing import Optional

from fastapi import FastAPI, HTTPException
from fastapi.responses import JSONResponse

from .dispatcher import KernelDispatcher
from .schemas import (ErrorResponse, KernelDetailResponse, KernelListResponse,
                      KernelRunRequest, KernelRunResponse)

logger = logging.getLogger(__name__)

_dispatcher: Optional[KernelDispatcher] = None


@asynccontextmanager
async def lifespan(app: FastAPI):
    global _dispatcher
    _dispatcher = KernelDispatcher(device="cuda")
    logger.info("kernel dispatcher ready on %s", _dispatcher.device)
    yield


app = FastAPI(title="Quantized GEMM kernel dispatch API (gfx950)", version="1.0.0",
              description="Invoke the MI355X quantized GEMM kernels by kernel_name + backend.",
              lifespan=lifespan)


@app.get("/health")
def health() -> dict:
    return {"status": "ok", "service": "kernel-dispatcher"}


@app.get("/api/v1/kernels", response_model=KernelListResponse)
def list_kernels() -> KernelListResponse:
    ks = _require_dispatcher().list_kernels()
    return KernelListResponse(count=len(ks), kernels=ks)


@app.get("/api/v1/kernels/{kernel_name}", response_model=KernelDetailResponse)
def kernel_detail(kernel_name: str, backend: str) -> KernelDetailResponse:
    d = _require_dispatcher()
    try:
        info = d.kernel_info(kernel_name, backend)
    except KeyError as exc:
        raise HTTPException(status_code=404, detail=str(exc)) from exc
    return KernelDetailResponse(**info, backends_available=d.list_backends(kernel_name))


def _error(status: int, kind: str, exc: Exception, req: KernelRunRequest) -> JSONResponse:
    body = ErrorResponse(error=kind, detail=str(exc), kernel_name=req.kernel_name,
                         backend=req.backend)
    return JSONResponse(status_code=status, content=body.model_dump())


@app.post("/api/v1/kernels/run", response_model=KernelRunResponse,
          responses={400: {"model": ErrorResponse}, 404: {"model": ErrorResponse}})
def run_kernel(req: KernelRunRequest):
    d = _require_dispatcher()
    try:
        res = d.run_from_spec(req.kernel_name, req.backend,
                              tensor_specs=[t.model_dump() for t in req.inputs],
                              scalar_params=req.params)
        return KernelRunResponse(**res.to_dict())
    except KeyError as exc:
        return _error(404, "kernel_not_found", exc, req)
    except Exception as exc:   # noqa: BLE001 -- every kernel failure maps to 400
        return _error(400, "kernel_dispatch_failed", exc, req)


def _require_dispatcher() -> KernelDispatcher:
    if _dispatcher is None:
        raise RuntimeError("Kernel dispatcher not initialised")
    return _dispatcher
