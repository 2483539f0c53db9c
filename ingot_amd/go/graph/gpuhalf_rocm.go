//go:build linux && amd64 && rocm && cgo

package graph

import "github.com/giraffesyo/ingot/kernels/rocm"

// GPUBF16 plan of the rocm session, the planHalf of the Metal session
// (graph/gpuhalf_darwin_arm64.go:29-112) restated for this backend's ops:
//
//   - a matrix product against a constant weight whose only consumer is an
//     activation node applies that activation in its store (fuseAct), and
//     the activation node passes its input through (actStep);
//   - a value read only by bf16 products against constant weights (as
//     their A operand, possibly through views) is produced in bf16 on the
//     device (halfOut): one f32 → bf16 pass less per consumer, the same
//     rounding the consumer's cast applies, so results do not change.
//
// A CPU node that reads such a value gets it widened back to f32 when it is
// downloaded (GPUSession.toHost).
func (s *GPUSession) planHalf() {
	type use struct{ step, slot int }
	users := make([][]use, s.nval)
	for i, st := range s.steps {
		for k, id := range st.in {
			if id >= 0 {
				users[id] = append(users[id], use{i, k})
			}
		}
	}
	n := len(s.steps)
	s.fuseAct, s.actStep, s.halfOut = make([]int, n), make([]bool, n), make([]bool, n)
	out0 := func(i int) int {
		if st := &s.steps[i]; len(st.out) > 0 {
			return st.out[0]
		}
		return -1
	}
	constWeight := func(st *step) bool {
		if len(st.in) < 2 || st.in[1] < 0 {
			return false
		}
		w := s.constVals[st.in[1]]
		return w != nil && w.Shape().Rank() == 2 && w.IsContiguous()
	}
	product := func(i int) bool {
		switch g := s.gops[i].(type) {
		case gemmGPU:
			return !g.transA && !g.quantI8
		case matmulGPU:
			return g.act == rocm.ActNone
		}
		return false
	}
	for i := range s.steps {
		st := &s.steps[i]
		id := out0(i)
		if !product(i) || !constWeight(st) || id < 0 || s.isOutput[id] || len(users[id]) != 1 || users[id][0].slot != 0 {
			continue
		}
		u := users[id][0].step
		if a, ok := s.gops[u].(unaryGPU); ok && out0(u) >= 0 {
			s.fuseAct[i], s.actStep[u] = a.act, true
		}
	}
	// want[id]: 0 unknown, 1 every consumer reads bf16, 2 not
	want := make([]int8, s.nval)
	var wants func(id int) bool
	reads := func(u use) bool {
		st := &s.steps[u.step]
		if st.node.Domain == "" && viewOps[st.node.OpType] {
			return u.slot == 0 && out0(u.step) >= 0 && wants(out0(u.step))
		}
		return u.slot == 0 && product(u.step) && constWeight(st) && !s.actStep[u.step]
	}
	wants = func(id int) bool {
		if want[id] == 0 {
			want[id] = 2 // provisional, ends cycles
			ok := !s.isOutput[id] && len(users[id]) > 0
			for _, u := range users[id] {
				if !ok {
					break
				}
				ok = reads(u)
			}
			if ok {
				want[id] = 1
			}
		}
		return want[id] == 1
	}
	for i := range s.steps {
		if !product(i) || !constWeight(&s.steps[i]) {
			continue
		}
		if id := out0(i); id >= 0 {
			if s.fuseAct[i] != 0 {
				// the value that flows on is the activation node's output
				s.halfOut[i] = wants(out0(users[id][0].step))
			} else {
				s.halfOut[i] = wants(id)
			}
		}
	}
}
