//go:build linux && amd64 && rocm && cgo

package graph

import "github.com/giraffesyo/ingot/kernels/rocm"

// The GPUBF16 plan of the rocm session: the decisions of the Metal session's
// planHalf (graph/gpuhalf_darwin_arm64.go:29-112), made here over this
// backend's ops.
//
//   - A matrix product against a constant weight whose output has exactly
//     one reader, an activation node reading it as its input, applies that
//     activation in its store (fuseAct); the activation node then passes its
//     input through (actStep).
//   - A value may live on the device as bf16 when it is not a graph output,
//     has readers, and every reader takes bf16 anyway: a product against a
//     constant weight reading it as its A operand, or a view whose own
//     output may live as bf16. Such a value is stored in bf16 by its
//     producer (halfOut): the rounding its readers' casts would apply, so
//     results do not change, and one f32 write and read less.
//
// A CPU node that reads such a value gets it widened back to f32 when it is
// downloaded (GPUSession.toHost).
func (s *GPUSession) planHalf() {
	n := len(s.steps)
	s.fuseAct, s.actStep, s.halfOut = make([]int, n), make([]bool, n), make([]bool, n)

	// Reader census: how many (step, slot) reads each value has, and the
	// last of them (the only one when the count is 1).
	reads := make([]int, s.nval)
	lastStep, lastSlot := make([]int, s.nval), make([]int, s.nval)
	for j := range s.steps {
		for k, id := range s.steps[j].in {
			if id >= 0 {
				reads[id]++
				lastStep[id], lastSlot[id] = j, k
			}
		}
	}
	firstOut := func(j int) int {
		if out := s.steps[j].out; len(out) > 0 {
			return out[0]
		}
		return -1
	}
	// bf16Product: step j is a matrix product whose A operand the bf16 math
	// takes, against a constant 2-D contiguous weight (input 1).
	bf16Product := func(j int) bool {
		switch g := s.gops[j].(type) {
		case gemmGPU:
			if g.transA || g.quantI8 {
				return false
			}
		case matmulGPU:
			if g.act != rocm.ActNone {
				return false
			}
		default:
			return false
		}
		in := s.steps[j].in
		if len(in) < 2 || in[1] < 0 {
			return false
		}
		w := s.constVals[in[1]]
		return w != nil && w.Shape().Rank() == 2 && w.IsContiguous()
	}

	for j := range s.steps {
		v := firstOut(j)
		if v < 0 || s.isOutput[v] || reads[v] != 1 || lastSlot[v] != 0 || !bf16Product(j) {
			continue
		}
		u := lastStep[v]
		if a, ok := s.gops[u].(unaryGPU); ok && firstOut(u) >= 0 {
			s.fuseAct[j] = a.act
			s.actStep[u] = true
		}
	}

	// halfOK[v]: value v may live as bf16. Every reader of a value comes
	// after its producer in the step order, so sweeping the steps backwards
	// settles a view's output before the view's own input is examined: each
	// read that does not take bf16 vetoes the value it reads.
	halfOK := make([]bool, s.nval)
	for v := range halfOK {
		halfOK[v] = reads[v] > 0 && !s.isOutput[v]
	}
	for j := n - 1; j >= 0; j-- {
		st := &s.steps[j]
		isView := st.node.Domain == "" && viewOps[st.node.OpType]
		for k, v := range st.in {
			if v < 0 || !halfOK[v] {
				continue
			}
			takes := false
			if k == 0 {
				if isView {
					w := firstOut(j)
					takes = w >= 0 && halfOK[w]
				} else {
					takes = bf16Product(j) && !s.actStep[j]
				}
			}
			if !takes {
				halfOK[v] = false
			}
		}
	}

	for j := range s.steps {
		if !bf16Product(j) {
			continue
		}
		v := firstOut(j)
		if v >= 0 && s.fuseAct[j] != 0 {
			v = firstOut(lastStep[v]) // the value that flows on is the activation node's output
		}
		s.halfOut[j] = v >= 0 && halfOK[v]
	}
}
