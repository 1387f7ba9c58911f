// Package hipnn runs the encoder forward of nn.(*Model).Forward
// (internal/nn/forward.go:129-245, inference) and decide.Local's per-call
// scoring on an AMD MI355X through libdecide_hip.so. The library is loaded at
// run time with purego, the way internal/cuda loads libcuda
// (internal/cuda/lib_unix.go:7-9, driver.go:62-105): no cgo, no ROCm headers
// at build time, and a machine without the library or a GPU gets ErrNoGPU so
// that callers fall back to the CPU as they do on cuda.ErrNoGPU
// (internal/train/engine.go:42-61).
//
// NOT COMPILED IN THIS REPOSITORY: its build image has no Go toolchain. What
// can be checked without one is checked from C and Python instead
// (tests/test_go_binding.py): every symbol this file registers is declared
// in include/decide_hip.h and exported by the library, the Go func types
// agree with the C prototypes, and tests/abi_replay.c dlopens the library
// with RTLD_NOW|RTLD_GLOBAL, resolves exactly these symbols and replays
// Load -> New -> Forward -> Free (dn_open's DN_NO_GPU -> ErrNoGPU on a
// machine without a GPU).
//
// Dependencies: github.com/ebitengine/purego (already in the reference's
// go.mod, v0.11.1) and the reference's internal/nn.
package hipnn

import (
	"errors"
	"fmt"
	"os"
	"runtime"
	"strconv"
	"strings"
	"sync"

	"github.com/ebitengine/purego"
	"github.com/jmwri/decide/internal/nn"
)

// ErrNoGPU is returned when the library, the HIP runtime or a device is
// missing: the counterpart of cuda.ErrNoGPU (internal/cuda/driver.go:19).
var ErrNoGPU = errors.New("hipnn: no usable AMD GPU / libdecide_hip.so found")

// Status codes of include/decide_hip.h.
const (
	dnOK          = 0
	dnNoGPU       = 1
	dnInvalidArg  = 2
	dnUnsupported = 5
)

// Precision of the device model (DN_PRECISION_*).
const (
	PrecisionFP32 int32 = 0 // fp32 MFMA everywhere: the validation mode
	PrecisionBF16 int32 = 1 // bf16 GEMM / attention operands, fp32 accumulation
	PrecisionFP16 int32 = 2 // binary16 operands (11-bit significands), fp32 accumulation
)

// DefaultCertifyMargin is the dn_set_certify margin the decide.Local wiring
// uses with PrecisionFP16: about 8x the fp16 forward's RMS error of a
// difference of two logits on ModernBERT-base (1.2e-4), so a question whose
// two best options are closer than that is answered from the fp32 path.
const DefaultCertifyMargin float32 = 1e-3

// Question kinds of dn_evaluate (DN_KIND_*), decide.Local's evalChoice /
// evalScore / evalNoul (local.go:264-356).
const (
	KindChoice int32 = 0
	KindScore  int32 = 1
	KindNoul   int32 = 2
)

type api struct {
	abiVersion   func() int32
	open         func(device int32, out *uintptr) int32
	close        func(ctx uintptr)
	lastError    func(ctx uintptr) string
	setConfig    func(ctx uintptr, hidden, inter, heads, layers, vocab int32, eps float32, halfWindow int32, thetaG, thetaL float64, sliding *uint8, precision int32) int32
	uploadTensor func(ctx uintptr, name string, data *float32, n int64) int32
	weightsReady func(ctx uintptr) int32
	setCertify   func(ctx uintptr, margin float32) int32
	forward      func(ctx uintptr, nseq int32, seqLen, ids, pos, optID, nmask, maskPos *int32, logits *float32, capacity int32) int32
	evaluate     func(ctx uintptr, nq int32, kind, nOpt, qLen, ids *int32, temperature *float64, maskID int32, independent int32, probs *float64, choice *int32, confidence, value *float64) int32
}

var (
	loadOnce sync.Once
	lib      api
	loadErr  error
)

// LibraryPath is the library Load opens: $DECIDE_HIP_LIBRARY, else the
// dynamic loader's search for libdecide_hip.so.
func LibraryPath() string {
	if p := os.Getenv("DECIDE_HIP_LIBRARY"); p != "" {
		return p
	}
	return "libdecide_hip.so"
}

// Load opens the library once. A missing library or entry point is ErrNoGPU.
func Load() error {
	loadOnce.Do(func() {
		h, err := purego.Dlopen(LibraryPath(), purego.RTLD_NOW|purego.RTLD_GLOBAL)
		if err != nil {
			loadErr = fmt.Errorf("%w (%v)", ErrNoGPU, err)
			return
		}
		missing := ""
		reg := func(fn any, sym string) {
			defer func() {
				if recover() != nil && missing == "" {
					missing = sym
				}
			}()
			purego.RegisterLibFunc(fn, h, sym)
		}
		reg(&lib.abiVersion, "dn_abi_version")
		reg(&lib.open, "dn_open")
		reg(&lib.close, "dn_close")
		reg(&lib.lastError, "dn_last_error")
		reg(&lib.setConfig, "dn_set_config")
		reg(&lib.uploadTensor, "dn_upload_tensor")
		reg(&lib.weightsReady, "dn_weights_ready")
		reg(&lib.setCertify, "dn_set_certify")
		reg(&lib.forward, "dn_forward")
		reg(&lib.evaluate, "dn_evaluate")
		if missing != "" {
			loadErr = fmt.Errorf("%w (library is missing %s)", ErrNoGPU, missing)
		}
	})
	return loadErr
}

// Model is a model resident on one GPU. Its methods may be called from any
// goroutine (every entry point selects the context's device itself) but not
// concurrently on one Model: callers serialise as decide.Local does with fmu.
type Model struct {
	ctx uintptr
}

// New opens device 0 and uploads m's tensors by their Tensors() names
// (internal/nn/model.go:51-84). It replaces cuda.Open + gpunn.New in
// train.NewInferer (internal/train/engine.go:152-167).
func New(m *nn.Model, precision int32) (*Model, error) {
	return NewWith(m, precision, 0)
}

// NewWith is New with certified argmax (dn_set_certify): with certifyMargin >
// 0 in a 16-bit precision, a sequence whose two largest logits are closer
// than the margin is recomputed on the library's fp32 twin, so its Choice
// comes out as the float32 reference's.
func NewWith(m *nn.Model, precision int32, certifyMargin float32) (*Model, error) {
	if err := Load(); err != nil {
		return nil, err
	}
	// Errors without a context are kept per OS thread by the library: read
	// dn_open's message on the thread that made the call.
	var ctx uintptr
	runtime.LockOSThread()
	rc := lib.open(0, &ctx)
	msg := ""
	if rc != dnOK {
		msg = lib.lastError(0)
	}
	runtime.UnlockOSThread()
	switch rc {
	case dnOK:
	case dnNoGPU:
		return nil, fmt.Errorf("%w (%s)", ErrNoGPU, msg)
	default:
		return nil, fmt.Errorf("hipnn: dn_open: %s", msg)
	}
	g := &Model{ctx: ctx}
	c := m.Cfg
	sliding := make([]uint8, c.Layers)
	for i := range sliding {
		if c.Sliding(i) {
			sliding[i] = 1
		}
	}
	var sp *uint8
	if len(sliding) > 0 {
		sp = &sliding[0]
	}
	if rc := lib.setConfig(ctx, int32(c.Hidden), int32(c.Intermediate), int32(c.Heads), int32(c.Layers),
		int32(c.Vocab), c.Eps, int32(c.HalfWindow), c.GlobalTheta, c.LocalTheta, sp, precision); rc != dnOK {
		err := g.err(rc)
		g.Free()
		return nil, err
	}
	if certifyMargin > 0 {
		if rc := lib.setCertify(ctx, certifyMargin); rc != dnOK {
			err := g.err(rc)
			g.Free()
			return nil, err
		}
	}
	for _, t := range m.Tensors() {
		if len(t.Data) == 0 {
			continue
		}
		if rc := lib.uploadTensor(ctx, t.Name, &t.Data[0], int64(len(t.Data))); rc != dnOK {
			err := g.err(rc)
			g.Free()
			return nil, err
		}
	}
	if lib.weightsReady(ctx) != 1 {
		g.Free()
		return nil, errors.New("hipnn: the model is missing tensors the device forward needs")
	}
	return g, nil
}

// err turns a status into the library's message. Input validation failures
// carry forward.go's own texts ("nn: sequence 0 has no options", ...).
func (g *Model) err(rc int32) error {
	msg := lib.lastError(g.ctx)
	if rc == dnInvalidArg {
		return errors.New(msg)
	}
	return fmt.Errorf("hipnn: %s (status %d)", msg, rc)
}

func ptr32(x []int32) *int32 {
	if len(x) == 0 {
		return nil
	}
	return &x[0]
}

// Forward has the contract of nn.(*Model).Forward(cache, batch, trainFrom >=
// Layers): one logit per mask position, in batch order.
func (g *Model) Forward(batch []nn.Sequence) ([]float32, error) {
	var seqLen, ids, pos, opt, nmask, maskPos []int32
	anyOpt := false
	for _, s := range batch {
		anyOpt = anyOpt || s.OptID != nil
	}
	for _, s := range batch {
		seqLen = append(seqLen, int32(len(s.IDs)))
		ids = append(ids, s.IDs...)
		pos = append(pos, s.Pos...)
		if anyOpt {
			if s.OptID != nil {
				opt = append(opt, s.OptID...)
			} else {
				for range s.IDs {
					opt = append(opt, -1)
				}
			}
		}
		nmask = append(nmask, int32(len(s.MaskPos)))
		for _, p := range s.MaskPos {
			maskPos = append(maskPos, int32(p))
		}
	}
	logits := make([]float32, len(maskPos))
	if len(batch) == 0 {
		return logits, nil
	}
	var out *float32
	if len(logits) > 0 {
		out = &logits[0]
	}
	if rc := lib.forward(g.ctx, int32(len(batch)), ptr32(seqLen), ptr32(ids), ptr32(pos), ptr32(opt), ptr32(nmask),
		ptr32(maskPos), out, int32(len(logits))); rc != dnOK {
		return nil, g.err(rc)
	}
	return logits, nil
}

// Question is one question of a SystemOne call as dn_evaluate takes it: the
// tokenizer's ids of bundle.PackText(state, instructions, options) with
// [CLS]/[SEP] (nil when a Choice or Score has at most one option), its
// option count and Calibration.TemperatureFor(kind).
type Question struct {
	Kind        int32
	NOpt        int32
	IDs         []int32
	Temperature float64
}

// Result is dn_evaluate's answer to one question.
type Result struct {
	Probs      []float64 // calibrated, rounded to 4 places
	Choice     int32     // argmax for a Choice, else -1
	Confidence float64   // marginConfidence for a Choice or Score
	Value      float64   // Score expectation (2 places) or Noul p(true) (4 places)
}

// QuestionError is a dn_evaluate failure of one question: Index is its
// position in the Evaluate call, Err the reason ("input contains the reserved
// [MASK] token", ...). decide.Local reports it under the question's id.
type QuestionError struct {
	Index int
	Err   error
}

func (e *QuestionError) Error() string { return fmt.Sprintf("decide: question %d: %v", e.Index, e.Err) }
func (e *QuestionError) Unwrap() error { return e.Err }

// questionError turns dn_evaluate's "decide: question N: reason" into a
// *QuestionError; other errors pass through.
func questionError(err error) error {
	const pre = "decide: question "
	msg := err.Error()
	if !strings.HasPrefix(msg, pre) {
		return err
	}
	num, reason, ok := strings.Cut(msg[len(pre):], ": ")
	idx, perr := strconv.Atoi(num)
	if !ok || perr != nil {
		return err
	}
	return &QuestionError{Index: idx, Err: errors.New(reason)}
}

// Evaluate answers every question of one call with a single forward: the
// batched form of Local.Evaluate's loop (local.go:126-150) over evalChoice /
// evalScore / evalNoul. Questions with at most one option (not Noul) carry
// no IDs and are answered without the model, as evalChoice / evalScore do. A
// failure of one question is a *QuestionError naming its index.
func (g *Model) Evaluate(qs []Question, maskID int32, independent bool) ([]Result, error) {
	n := len(qs)
	if n == 0 {
		return nil, nil
	}
	kind, nOpt, qLen := make([]int32, n), make([]int32, n), make([]int32, n)
	temp := make([]float64, n)
	var ids []int32
	total := 0
	for i, q := range qs {
		kind[i], nOpt[i], qLen[i], temp[i] = q.Kind, q.NOpt, int32(len(q.IDs)), q.Temperature
		ids = append(ids, q.IDs...)
		total += int(q.NOpt)
	}
	probs := make([]float64, total+1)
	choice := make([]int32, n)
	conf, value := make([]float64, n), make([]float64, n)
	ind := int32(0)
	if independent {
		ind = 1
	}
	if rc := lib.evaluate(g.ctx, int32(n), &kind[0], &nOpt[0], &qLen[0], ptr32(ids), &temp[0], maskID, ind,
		&probs[0], &choice[0], &conf[0], &value[0]); rc != dnOK {
		return nil, questionError(g.err(rc))
	}
	out := make([]Result, n)
	off := 0
	for i := range qs {
		k := int(nOpt[i])
		out[i] = Result{Probs: append([]float64(nil), probs[off:off+k]...), Choice: choice[i],
			Confidence: conf[i], Value: value[i]}
		off += k
	}
	return out, nil
}

// Free releases the device model (gpunn.(*Model).Free + cuda.(*Device).Close).
func (g *Model) Free() {
	if g.ctx != 0 {
		lib.close(g.ctx)
		g.ctx = 0
	}
}
