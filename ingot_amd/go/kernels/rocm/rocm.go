//go:build linux && amd64 && rocm && cgo

// Package rocm binds libingot_rocm, the MI355X (gfx950) kernels of ingot's
// dense-contraction path: Gemm / MatMul with fused bias and activation
// epilogues, bf16-weight GEMM and decode GEMV, int8 MatMulInteger with fused
// DequantizeLinear, QLinearMatMul and QLinearConv. It is the ROCm
// counterpart of kernels/metal: plain device pointers and sizes cross the
// boundary, every call is enqueued on the session's HIP stream, and Sync
// waits for it. The graph package's rocm GPUSession (graph/gpu_rocm.go) is
// its only caller.
//
// Build: the library and its header come from the ingot-rocm tree
// (python ingot_amd/build.py); point cgo at them with
//
//	CGO_CFLAGS=-I<ingot-rocm>/include CGO_LDFLAGS="-L<ingot-rocm>/ingot_amd -lingot_rocm -Wl,-rpath,<ingot-rocm>/ingot_amd"
//
// and build with -tags rocm.
package rocm

/*
#cgo LDFLAGS: -lingot_rocm
#include <stdlib.h>
#include "ingot_rocm.h"
*/
import "C"

import (
	"errors"
	"fmt"
	"runtime"
	"unsafe"
)

// Status codes of the C ABI (include/ingot_rocm.h).
const (
	statusOK       = 0
	statusInval    = 1
	statusDeclined = 2
	statusDevice   = 3
	statusNoMem    = 4
)

// ErrDeclined is INGOT_EDECLINED: the inputs are valid for the op but the
// GPU does not run them; the caller runs the CPU op (gpuOp.prepare's
// ok = false in the Metal backend, graph/gpuops_darwin_arm64.go:14-22).
var ErrDeclined = errors.New("rocm: declined")

// Error is a failed library call: the status code and the library's message.
type Error struct {
	Code int
	Msg  string
}

func (e *Error) Error() string { return fmt.Sprintf("rocm: %s (status %d)", e.Msg, e.Code) }

// Is makes errors.Is(err, ErrDeclined) true for declined calls.
func (e *Error) Is(target error) bool { return target == ErrDeclined && e.Code == statusDeclined }

// call runs one library function. The library keeps its last error per OS
// thread, so the call and its ingot_rocm_last_error run on one thread.
func call(f func() C.int) error {
	runtime.LockOSThread()
	defer runtime.UnlockOSThread()
	rc := f()
	if rc == statusOK {
		return nil
	}
	return &Error{Code: int(rc), Msg: C.GoString(C.ingot_rocm_last_error())}
}

// DType codes: the numbering of tensor.DType (tensor/dtype.go:12-23).
const (
	F32  = 1
	F16  = 2
	BF16 = 3
	I8   = 4
	U8   = 5
	I16  = 6
	I32  = 7
	I64  = 8
	Bool = 9
	// PackI8G packs a weight as int8 with one f32 scale per 64 k of a row
	// (ingot_weight_quant="int8", kernels/gemm/i8g.go:12-56).
	PackI8G = 100
)

// Epilogue activations (INGOT_ACT_*; ops/epilogue.go:22-73 and the Metal
// set, kernels/metal/cnn.go:15-37).
const (
	ActNone        = 0
	ActRelu        = 1
	ActGeluErf     = 2
	ActGeluTanh    = 3
	ActSigmoid     = 4
	ActSiLU        = 5
	ActHardSwish   = 6
	ActHardSigmoid = 7
	ActClip        = 8
	ActLeakyRelu   = 9
)

// Gemm C operand broadcast (ops/matmul.go:50-76).
const (
	CNone   = 0
	CFull   = 1
	CRow    = 2
	CCol    = 3
	CScalar = 4
)

// Math type of a product.
const (
	MathAuto = 0
	MathF32  = 1
	MathBF16 = 2
)

// DevPtr is device memory of the session's GPU (never Go memory).
type DevPtr unsafe.Pointer

// At is p advanced by off bytes.
func (p DevPtr) At(off int) DevPtr { return DevPtr(unsafe.Add(unsafe.Pointer(p), off)) }

// Session is one device's stream, device pool and weight table
// (ingot_rocm_open).
type Session struct {
	h *C.ingot_rocm_session
}

// Open opens a session on HIP device dev.
func Open(dev int) (*Session, error) {
	s := &Session{}
	if err := call(func() C.int { return C.ingot_rocm_open(C.int(dev), &s.h) }); err != nil {
		return nil, err
	}
	return s, nil
}

// Close waits for queued work and frees the session's weights, buffers and
// stream.
func (s *Session) Close() error {
	if s == nil || s.h == nil {
		return nil
	}
	err := call(func() C.int { return C.ingot_rocm_close(s.h) })
	s.h = nil
	return err
}

// Sync waits for every call enqueued on the session; GPU faults surface here.
func (s *Session) Sync() error { return call(func() C.int { return C.ingot_rocm_sync(s.h) }) }

// Alloc returns n bytes of device memory.
func (s *Session) Alloc(n int) (DevPtr, error) {
	var p unsafe.Pointer
	err := call(func() C.int { return C.ingot_rocm_device_alloc(s.h, C.size_t(n), &p) })
	return DevPtr(p), err
}

// Free releases Alloc'd memory (after the queued work that uses it).
func (s *Session) Free(p DevPtr) error {
	return call(func() C.int { return C.ingot_rocm_device_free(s.h, unsafe.Pointer(p)) })
}

// HostAlloc returns n bytes of pinned host memory, the backing a
// tensor.NewPoolAlloc pool can use (tensor/pool.go:22).
func (s *Session) HostAlloc(n int) ([]byte, error) {
	var p unsafe.Pointer
	if err := call(func() C.int { return C.ingot_rocm_host_alloc(s.h, C.size_t(n), &p) }); err != nil {
		return nil, err
	}
	return unsafe.Slice((*byte)(p), n), nil
}

// HostFree releases HostAlloc'd memory.
func (s *Session) HostFree(b []byte) error {
	if len(b) == 0 {
		return nil
	}
	return call(func() C.int { return C.ingot_rocm_host_free(s.h, unsafe.Pointer(&b[0])) })
}

// Upload copies src to device memory and returns when it has arrived (so
// the C side keeps no Go pointer).
func (s *Session) Upload(dst DevPtr, src []byte) error {
	if len(src) == 0 {
		return nil
	}
	return call(func() C.int {
		return C.ingot_rocm_memcpy_h2d(s.h, unsafe.Pointer(dst), unsafe.Pointer(&src[0]), C.size_t(len(src)))
	})
}

// Download copies device memory to dst after the queued work has finished.
func (s *Session) Download(dst []byte, src DevPtr) error {
	if len(dst) == 0 {
		return nil
	}
	return call(func() C.int {
		return C.ingot_rocm_memcpy_d2h(s.h, unsafe.Pointer(&dst[0]), unsafe.Pointer(src), C.size_t(len(dst)))
	})
}

// Copy copies n bytes between device buffers.
func (s *Session) Copy(dst, src DevPtr, n int) error {
	return call(func() C.int {
		return C.ingot_rocm_memcpy_d2d(s.h, unsafe.Pointer(dst), unsafe.Pointer(src), C.size_t(n))
	})
}

// TimerStart records a timing event on the stream; TimerStop records a
// second one, waits for it and returns the GPU time between them.
func (s *Session) TimerStart() error { return call(func() C.int { return C.ingot_rocm_timer_start(s.h) }) }

func (s *Session) TimerStop() (float32, error) {
	var ms C.float
	err := call(func() C.int { return C.ingot_rocm_timer_stop(s.h, &ms) })
	return float32(ms), err
}

// Weight is a constant weight packed once on the device (bCache /
// bf16Const / bWeights: ops/matmul.go:200-236,
// graph/gpuops_darwin_arm64.go:610-629, ops/quant.go:803-829).
type Weight struct {
	h    *C.ingot_rocm_weight
	N, K int
}

// UploadWeight packs a host weight. trans: the source is [N,K] (rows = N);
// else [K,N]. src holds rows×cols elements of srcDType, row pitch cols.
func (s *Session) UploadWeight(srcDType, packDType, rows, cols int, trans bool, src []byte) (*Weight, error) {
	if len(src) == 0 {
		return nil, &Error{Code: statusInval, Msg: "empty weight"}
	}
	w := &Weight{}
	tr := C.int(0)
	if trans {
		tr = 1
	}
	err := call(func() C.int {
		return C.ingot_rocm_weight_upload(s.h, C.int(srcDType), C.int(packDType), C.int64_t(rows), C.int64_t(cols),
			C.int64_t(cols), tr, unsafe.Pointer(&src[0]), &w.h)
	})
	if err != nil {
		return nil, err
	}
	var n, k C.int64_t
	var dt C.int
	if err := call(func() C.int { return C.ingot_rocm_weight_info(w.h, &n, &k, &dt) }); err != nil {
		return nil, err
	}
	w.N, w.K = int(n), int(k)
	return w, nil
}

// PackWeight packs a weight already in device memory (a per-call pack).
func (s *Session) PackWeight(srcDType, packDType, rows, cols int, trans bool, src DevPtr) (*Weight, error) {
	w := &Weight{}
	tr := C.int(0)
	if trans {
		tr = 1
	}
	err := call(func() C.int {
		return C.ingot_rocm_weight_pack_device(s.h, C.int(srcDType), C.int(packDType), C.int64_t(rows),
			C.int64_t(cols), C.int64_t(cols), tr, unsafe.Pointer(src), &w.h)
	})
	if err != nil {
		return nil, err
	}
	if trans {
		w.N, w.K = rows, cols
	} else {
		w.N, w.K = cols, rows
	}
	return w, nil
}

// FreeWeight releases a packed weight.
func (s *Session) FreeWeight(w *Weight) error {
	if w == nil || w.h == nil {
		return nil
	}
	err := call(func() C.int { return C.ingot_rocm_weight_free(s.h, w.h) })
	w.h = nil
	return err
}

// Gemm is one product Y = post_scale·act(alpha·op(A)·Bᵀ + beta·C) + post_shift
// (ingot_rocm_gemm_args).
type Gemm struct {
	M, N, K         int
	A               DevPtr
	ADType          int // F32 or BF16
	TransA          bool
	LDA             int
	W               *Weight // nil for GemmDynamicB
	Alpha, Beta     float32
	C               DevPtr
	CMode           int
	Math            int
	LDC             int
	Act             int
	ActAlpha        float32
	ActBeta         float32
	Post            bool
	PostScale       float32
	PostShift       float32
	Y               DevPtr
	LDY             int
	YDType          int // F32 (or 0) or BF16
	Batch           int
	StrideA, StrideY int // elements between batch items
}

func (g *Gemm) args() C.ingot_rocm_gemm_args {
	var a C.ingot_rocm_gemm_args
	a.M, a.N, a.K = C.int64_t(g.M), C.int64_t(g.N), C.int64_t(g.K)
	a.d_a = unsafe.Pointer(g.A)
	a.a_dtype = C.int32_t(g.ADType)
	if g.TransA {
		a.trans_a = 1
	}
	a.lda = C.int64_t(g.LDA)
	if g.W != nil {
		a.w = g.W.h
	}
	a.alpha, a.beta = C.float(g.Alpha), C.float(g.Beta)
	a.d_c = (*C.float)(unsafe.Pointer(g.C))
	a.c_mode = C.int32_t(g.CMode)
	a.math = C.int32_t(g.Math)
	a.ldc = C.int64_t(g.LDC)
	a.act = C.int32_t(g.Act)
	a.act_alpha, a.act_beta = C.float(g.ActAlpha), C.float(g.ActBeta)
	if g.Post {
		a.post = 1
	}
	a.post_scale, a.post_shift = C.float(g.PostScale), C.float(g.PostShift)
	a.d_y = (*C.float)(unsafe.Pointer(g.Y))
	a.ldy = C.int64_t(g.LDY)
	a.batch = C.int64_t(max(g.Batch, 1))
	a.stride_a, a.stride_y = C.int64_t(g.StrideA), C.int64_t(g.StrideY)
	a.y_dtype = C.int32_t(g.YDType)
	return a
}

// Gemm enqueues the product against the packed weight g.W (ingot_rocm_gemm).
func (s *Session) Gemm(g *Gemm) error {
	a := g.args()
	return call(func() C.int { return C.ingot_rocm_gemm(s.h, &a) })
}

// GemmNoAlloc is Gemm with its scratch in the library's fixed per-GPU array
// (ingot_rocm_gemm_noalloc): for callers that must not allocate.
func (s *Session) GemmNoAlloc(g *Gemm) error {
	a := g.args()
	return call(func() C.int { return C.ingot_rocm_gemm_noalloc(s.h, &a) })
}

// GemmDynamicB enqueues a (batched) product whose B is an activation in
// device memory: [N,K] items when transB (attention Q·Kᵀ), else [K,N]
// (ingot_rocm_gemm_dynamic_b; matmulOp's batched path, ops/matmul.go:375-403).
func (s *Session) GemmDynamicB(g *Gemm, b DevPtr, bDType int, transB bool, ldb, strideB int) error {
	a := g.args()
	tb := C.int32_t(0)
	if transB {
		tb = 1
	}
	return call(func() C.int {
		return C.ingot_rocm_gemm_dynamic_b(s.h, &a, unsafe.Pointer(b), C.int32_t(bDType), tb, C.int64_t(ldb),
			C.int64_t(strideB))
	})
}

// GemvBF16 enqueues the decode GEMV for M <= 16 rows (ingot_rocm_gemv_bf16).
func (s *Session) GemvBF16(g *Gemm) error {
	a := g.args()
	return call(func() C.int { return C.ingot_rocm_gemv_bf16(s.h, &a) })
}

// MatMulInteger enqueues Y_i32 = Σ (A − za)·B (exact) and/or its fused
// dequantisation Y_f32 = float32(Y_i32 − dqZp)·scale[n or 0]
// (ingot_rocm_matmul_integer; ops/quant.go:831-900,173-229).
func (s *Session) MatMulInteger(m, n, k int, a DevPtr, aDType, lda int, za int32, w *Weight, yI32 DevPtr,
	scale DevPtr, nScale int, dqZp int32, yF32 DevPtr) error {
	return call(func() C.int {
		return C.ingot_rocm_matmul_integer(s.h, C.int64_t(m), C.int64_t(n), C.int64_t(k), unsafe.Pointer(a),
			C.int32_t(aDType), C.int64_t(lda), C.int32_t(za), w.h, (*C.int32_t)(unsafe.Pointer(yI32)),
			(*C.float)(unsafe.Pointer(scale)), C.int64_t(nScale), C.int32_t(dqZp), (*C.float)(unsafe.Pointer(yF32)))
	})
}

// QLinearMatMul enqueues the requantised int8 product (ops/quant.go:902-928).
func (s *Session) QLinearMatMul(m, n, k int, a DevPtr, aDType, lda int, za int32, w *Weight, mult float32, zy int32,
	yDType int, y DevPtr) error {
	return call(func() C.int {
		return C.ingot_rocm_qlinear_matmul(s.h, C.int64_t(m), C.int64_t(n), C.int64_t(k), unsafe.Pointer(a),
			C.int32_t(aDType), C.int64_t(lda), C.int32_t(za), w.h, C.float(mult), C.int32_t(zy), C.int32_t(yDType),
			unsafe.Pointer(y))
	})
}

// DequantizeLinear enqueues y[i] = float32(x[i] − zp[c])·scale[c],
// c = (i / inner) % nScale (ops/quant.go:173-229). zp may be nil.
func (s *Session) DequantizeLinear(x DevPtr, xDType, n int, scale DevPtr, nScale, inner int, zp DevPtr, zpDType,
	nZp int, y DevPtr) error {
	return call(func() C.int {
		return C.ingot_rocm_dequantize_linear(s.h, unsafe.Pointer(x), C.int32_t(xDType), C.int64_t(n),
			(*C.float)(unsafe.Pointer(scale)), C.int64_t(nScale), C.int64_t(inner), unsafe.Pointer(zp),
			C.int32_t(zpDType), C.int64_t(nZp), (*C.float)(unsafe.Pointer(y)))
	})
}

// Activation enqueues y = act(x + bias[col]) over rows×cols f32 values (the
// standalone Relu / Gelu nodes, ops/elementwise.go:492,533-539). bias may be nil.
func (s *Session) Activation(x, y DevPtr, rows, cols int, bias DevPtr, act int, actAlpha, actBeta float32) error {
	return call(func() C.int {
		return C.ingot_rocm_activation(s.h, (*C.float)(unsafe.Pointer(x)), (*C.float)(unsafe.Pointer(y)),
			C.int64_t(rows), C.int64_t(cols), (*C.float)(unsafe.Pointer(bias)), C.int32_t(act), C.float(actAlpha),
			C.float(actBeta), 0, 1, 0)
	})
}

// CastBF16 enqueues y = bf16(x) (RNE) over n values (kernels/gemm/bgemm.go:20-26).
func (s *Session) CastBF16(x, y DevPtr, n int) error {
	return call(func() C.int {
		return C.ingot_rocm_cast_bf16(s.h, (*C.float)(unsafe.Pointer(x)), (*C.uint16_t)(unsafe.Pointer(y)),
			C.int64_t(n))
	})
}
