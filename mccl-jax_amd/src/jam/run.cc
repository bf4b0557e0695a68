#include "jam/run.h"

#include <cstdio>
#include <cstring>
#include <mutex>

#include "mk_kernels.h"

namespace mi::jam {

std::vector<void*>* Program::DeviceConsts(int ordinal) {
  std::lock_guard<std::mutex> lk(mu_);
  if (dev_consts_.size() <= size_t(ordinal)) dev_consts_.resize(ordinal + 1);
  auto& v = dev_consts_[ordinal];
  if (v.size() == consts.size()) return &v;
  std::string err;
  exec::DeviceContext* dev = exec::DeviceContext::Get(ordinal, &err);
  if (!dev) return nullptr;
  for (size_t i = v.size(); i < consts.size(); ++i) {
    void* p = dev->Alloc(consts[i].bytes.size(), &err);
    if (!p && !consts[i].bytes.empty()) return nullptr;
    if (!dev->UploadForCompute(p, consts[i].bytes.data(), consts[i].bytes.size(), &err)) return nullptr;
    v.push_back(p);
  }
  return &v;
}

Program::~Program() {
  for (size_t o = 0; o < dev_consts_.size(); ++o) {
    if (dev_consts_[o].empty()) continue;
    exec::DeviceContext* dev = exec::DeviceContext::Get(int(o), nullptr);
    if (!dev) continue;
    for (void* p : dev_consts_[o]) dev->Free(p);
  }
}

namespace {

struct Frame {
  const std::vector<RunInput>* inputs;
  std::vector<RunOutput>* outputs;
  std::vector<void*>* consts;
  char* arena;
  const EwJit* jit;          // generated ew kernels of the plan (null: none)
  void* const* jit_fns;      // their hipFunction_t handles on this device (null: interpreter)
  std::string* error;        // message of a failure not reported through mk_last_error
};

void* Resolve(const BufRef& b, const Frame& f) {
  switch (b.space) {
    case Space::kInput: return const_cast<char*>(static_cast<const char*>((*f.inputs)[b.index].data)) + b.offset;
    case Space::kOutput: return static_cast<char*>((*f.outputs)[b.index].data) + b.offset;
    case Space::kArena: return f.arena + b.offset;
    case Space::kConst: return static_cast<char*>((*f.consts)[b.index]) + b.offset;
    case Space::kNone: return nullptr;
  }
  return nullptr;
}

// Step encodings (written by lower.cc):
//   gemm     bufs A,B,C[,bias[,Y]]  i ab_type,c_type,batch,M,N,K,a_bs,a_ms,a_ks,b_bs,b_ks,b_ns,c_bs,c_ms,epilogue
//                               [,y_ms]  (Y: bf16 gelu_tanh of C, mk_gemm_bias_gelu)
//   gemm_blas bufs A,B,C        i as gemm (no epilogue)
//   gemm_splitk bufs A,B,C,workspace[,bias]  i ab_type,M,N,K,a_ms,a_ks,b_ks,b_ns,c_ms,splits,epilogue
//   sdpa     bufs Q,K,V,O[,lse] i B,H,Sq,Sk,D,q_bs,q_hs,q_ss,k_bs,k_hs,k_ss,v_bs,v_hs,v_ss,o_bs,o_hs,o_ss,causal  f scale
//   row_reduce bufs x,y         i in_type,out_type,op,rows,cols  f init
//   argmax   bufs x,values,idx  i in_type,is_min,rows,cols,index_type,has_values
//   layernorm bufs x,g,b,y[,x2,xsum]  i out_type,rows,cols[,in_type]  f eps (x2: x + x2 normalised, stored to xsum)
//   layernorm_bwd bufs x,g,dy,dres,dx,dgamma,dbeta,dx_colsum,workspace[,dx_bf16]  i io_type,rows,cols  f eps
//   gelu     bufs x,y           i io_type,n
//   ew       bufs in...,out...  i rank,dims[6],n_inputs,(out_reg,out_type) per output  prog  strides[6n]
//                               types[n]  f consts  (batch > 1: bufs of each instance in turn)
//   gather   bufs table,ids,out i n_rows,row_bytes,index_type,n_ids
//   scatter_add bufs table,ids,updates,out,workspace  i dtype,n_rows,row_len,index_type,n_ids
//   iota     bufs out           i out_type,rank,dim,dims...
//   copy_strided bufs in,out    i elem_bytes,rank,dims...  strides
//   softmax  bufs x,y           i io_type,rows,cols
//   softmax_xent bufs logits,labels,loss_rows,dlogits  i logits_type,rows,cols,label_type,dlogits_type,
//                               ld_logits,ld_dlogits  f grad_scale
//   sdpa_bwd bufs q,k,v,o,dout,lse,dq,dk,dv,workspace
//            i B,H,Sq,Sk,D, (b,h,s strides) of q,k,v,o,dout,dq,dk,dv, causal  f scale
//   ew_reduce bufs in...,out,tmp,ws[,stored]  i rank,dims[6],n_inputs,out_reg,val_type,out_type,rop,
//                               rows,cols,mode,init bits,store  prog strides types f as ew (mode 0: reduce
//                               trailing dims, mode 1: sum leading dims; store 1 / 2: the value also
//                               into `stored`, as val_type / bf16)
//   convert  bufs in,out        i in_type,out_type,n
//   fill     bufs out           i elem_bytes,n,pattern
//   copy     bufs in,out        i bytes
int RunStep(const Step& s, const Frame& f, hipStream_t stream) {
  void* st = reinterpret_cast<void*>(stream);
  auto P = [&](size_t k) { return Resolve(s.bufs[k], f); };
  const auto& i = s.i;
  switch (s.kind) {
    case StepKind::kGemm:
      if (s.bufs.size() > 4)  // + the GELU side output (bufs 4, rows i[15] apart)
        return mk_gemm_bias_gelu(st, int(i[0]), int(i[1]), i[3], i[4], i[5], P(0), i[7], i[8], P(1), i[10], i[11],
                                 P(2), i[13], P(3), int(i[14]), P(4), i[15]);
      return mk_gemm(st, int(i[0]), int(i[1]), i[2], i[3], i[4], i[5], P(0), i[6], i[7], i[8], P(1), i[9],
                     i[10], i[11], P(2), i[12], i[13], s.bufs.size() > 3 ? P(3) : nullptr, int(i[14]));
    case StepKind::kSdpa:
      return mk_sdpa_fwd(st, i[0], i[1], i[2], i[3], i[4], P(0), i[5], i[6], i[7], P(1), i[8], i[9], i[10],
                         P(2), i[11], i[12], i[13], P(3), i[14], i[15], i[16], s.f[0], int(i[17]),
                         s.bufs.size() > 4 ? static_cast<float*>(P(4)) : nullptr);
    case StepKind::kSoftmaxXent:
      return mk_softmax_xent_strided(st, int(i[0]), int(i[4]), i[1], i[2], P(0), i[5], int(i[3]), P(1), s.f[0],
                                     static_cast<float*>(P(2)), P(3), i[6]);
    case StepKind::kGemmBlas:
      return mk_gemm_blas(st, int(i[0]), int(i[1]), i[2], i[3], i[4], i[5], P(0), i[6], i[7], i[8], P(1), i[9],
                          i[10], i[11], P(2), i[12], i[13], 1.f, 0.f);
    case StepKind::kSdpaBwd:
      return mk_sdpa_bwd(st, i[0], i[1], i[2], i[3], i[4], P(0), i[5], i[6], i[7], P(1), i[8], i[9], i[10],
                         P(2), i[11], i[12], i[13], P(3), i[14], i[15], i[16], P(4), i[17], i[18], i[19],
                         static_cast<const float*>(P(5)), P(6), i[20], i[21], i[22], P(7), i[23], i[24], i[25],
                         P(8), i[26], i[27], i[28], s.f[0], int(i[29]), P(9));
    case StepKind::kGemmSplitK:
      return mk_gemm_splitk_typed(st, int(i[0]), MK_F32, i[1], i[2], i[3], P(0), i[4], i[5], P(1), i[6], i[7], P(2),
                                  i[8], i[9], P(3), s.bufs.size() > 4 ? P(4) : nullptr, int(i[10]));
    case StepKind::kColSum:  // y[c] = sum_r x[r, c]: i = {dtype, rows, cols}
      return mk_col_sum(st, int(i[0]), i[1], i[2], P(0), static_cast<float*>(P(1)), P(2));
    case StepKind::kRowReduce:
      return mk_row_reduce(st, int(i[0]), int(i[1]), int(i[2]), i[3], i[4], P(0), s.f[0], P(1));
    case StepKind::kArgmax:
      return mk_row_argmax(st, int(i[0]), int(i[1]), i[2], i[3], P(0), i[5] ? P(1) : nullptr, int(i[4]), P(2));
    case StepKind::kLayerNorm:
      if (s.bufs.size() > 4)  // x = bufs 0 + bufs 4, stored to bufs 5
        return mk_add_layernorm_typed(st, int(i[3]), int(i[0]), i[1], i[2], P(0), P(4), nullptr, P(1), P(2), s.f[0],
                                      P(5), P(3));
      if (i.size() > 3) return mk_layernorm_typed(st, int(i[3]), int(i[0]), i[1], i[2], P(0), P(1), P(2), s.f[0], P(3));
      return mk_layernorm(st, int(i[0]), i[1], i[2], P(0), P(1), P(2), s.f[0], P(3));
    case StepKind::kLayerNormBwd:
      return mk_layernorm_bwd_typed(st, int(i[0]), i[1], i[2], P(0), P(1), P(2), P(3), s.f[0], P(4),
                                    s.bufs.size() > 9 ? P(9) : nullptr, static_cast<float*>(P(5)),
                                    static_cast<float*>(P(6)), static_cast<float*>(P(7)), P(8));
    case StepKind::kGelu:
      return mk_gelu_tanh(st, int(i[0]), i[1], P(0), P(1));
    case StepKind::kEw: {
      const int n_in = int(i[7]);
      const int per = s.batch > 0 ? int(s.bufs.size()) / s.batch : 0;
      const int n_out = per - n_in;
      if (n_in > 8 || n_out < 1 || n_out > 4 || per * s.batch != int(s.bufs.size())) return MK_ERR_INVALID;
      if (s.jit >= 0 && f.jit_fns) {
        // the step's generated kernel, when every pointer has the alignment
        // its vector accesses assume (otherwise the interpreter below); a
        // batched kernel takes every instance's pointers in one struct
        const EwKernel& k = f.jit->kernel(s.jit);
        const int pi = n_in > 0 ? n_in : 1;
        void* ptrs[kEwJitMaxBatch * 13];
        bool aligned = (k.batch == 0 ? s.batch == 1 : k.batch == s.batch) && k.n_in == n_in && k.n_out == n_out;
        for (int inst = 0; aligned && inst < s.batch; ++inst)
          for (int b = 0; aligned && b < per; ++b) {
            void* ptr = P(size_t(inst * per + b));
            aligned = reinterpret_cast<uintptr_t>(ptr) % k.align[size_t(b)] == 0;
            if (k.batch == 0) ptrs[b] = ptr;
            else if (b < n_in) ptrs[inst * pi + b] = ptr;
            else ptrs[s.batch * pi + inst * n_out + (b - n_in)] = ptr;
          }
        if (aligned) {
          void* args[16];
          if (k.batch == 0)
            for (int b = 0; b < per; ++b) args[b] = &ptrs[b];
          else
            args[0] = ptrs;
          hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(f.jit_fns[2 * s.jit]), k.blocks * uint32_t(s.batch),
                                               1, 1, kEwJitBlock, 1, 1, 0, stream, args, nullptr);
          if (e == hipSuccess) return MK_OK;
          *f.error = "hipModuleLaunchKernel(" + k.name + "): " + hipGetErrorString(e);
          return MK_ERR_LAUNCH;
        }
        if (f.jit->strict) {
          *f.error = "generated kernel " + k.name + ": a buffer misses its alignment (strict mode)";
          return MK_ERR_INVALID;
        }
      }
      for (int inst = 0; inst < s.batch; ++inst) {
        const void* ins[8];
        int types[8];
        for (int k = 0; k < n_in; ++k) {
          ins[k] = P(size_t(inst * per + k));
          types[k] = s.types[size_t(k)];
        }
        int regs[4], otypes[4];
        void* outs[4];
        for (int k = 0; k < n_out; ++k) {
          regs[k] = int(i[8 + 2 * size_t(k)]);
          otypes[k] = int(i[9 + 2 * size_t(k)]);
          outs[k] = P(size_t(inst * per + n_in + k));
        }
        const int rc = mk_ew_program_multi(st, int(i[0]), &i[1], n_in, ins, types, s.strides.data(),
                                           int(s.prog.size() / 4), s.prog.data(), s.f.data(), int(s.f.size()), n_out,
                                           regs, otypes, outs);
        if (rc != MK_OK) return rc;
      }
      return MK_OK;
    }
    case StepKind::kEwReduce: {
      const int n_in = int(i[7]);
      const bool store = i.size() == 17 && i[16] != 0;
      if (n_in > 8 || s.bufs.size() != size_t(n_in + (store ? 4 : 3)) || i.size() != 17) return MK_ERR_INVALID;
      const int mode = int(i[14]);
      if (s.jit >= 0 && f.jit_fns) {
        // generated: the reduction reads the program's inputs (mode 1: then
        // adds the row chunks' partial sums from the workspace)
        const EwKernel& k = f.jit->kernel(s.jit);
        void* ptrs[10];
        bool aligned = k.n_in == n_in;
        for (int b = 0; aligned && b < n_in; ++b) {
          ptrs[b] = P(size_t(b));
          aligned = reinterpret_cast<uintptr_t>(ptrs[b]) % k.align[size_t(b)] == 0;
        }
        if (store) aligned = aligned && reinterpret_cast<uintptr_t>(P(size_t(n_in + 3))) % k.align[size_t(n_in + 3)] == 0;
        if (aligned) {
          ptrs[n_in] = k.kind == 1 ? P(size_t(n_in)) : P(size_t(n_in + 2));
          if (store) ptrs[n_in + 1] = P(size_t(n_in + 3));
          void* args[10];
          for (int b = 0; b <= n_in + (store ? 1 : 0); ++b) args[b] = &ptrs[b];
          hipError_t e = hipModuleLaunchKernel(static_cast<hipFunction_t>(f.jit_fns[2 * s.jit]), k.blocks, 1, 1,
                                               kEwJitBlock, 1, 1, 0, stream, args, nullptr);
          if (e == hipSuccess && k.kind == 2) {
            void* fp[2] = {P(size_t(n_in + 2)), P(size_t(n_in))};
            void* fa[2] = {&fp[0], &fp[1]};
            e = hipModuleLaunchKernel(static_cast<hipFunction_t>(f.jit_fns[2 * s.jit + 1]), k.final_blocks, 1, 1,
                                      kEwJitBlock, 1, 1, 0, stream, fa, nullptr);
          }
          if (e == hipSuccess) return MK_OK;
          *f.error = "hipModuleLaunchKernel(" + k.name + "): " + hipGetErrorString(e);
          return MK_ERR_LAUNCH;
        }
        if (f.jit->strict) {
          *f.error = "generated kernel " + k.name + ": a buffer misses its alignment (strict mode)";
          return MK_ERR_INVALID;
        }
      }
      // interpreter: the value into tmp, then the library's reduction
      const void* ins[8];
      int types[8];
      for (int k = 0; k < n_in; ++k) {
        ins[k] = P(size_t(k));
        types[k] = s.types[size_t(k)];
      }
      int reg = int(i[8]), vt = int(i[9]);
      void* tmp = P(size_t(n_in + 1));
      int rc = mk_ew_program_multi(st, int(i[0]), &i[1], n_in, ins, types, s.strides.data(), int(s.prog.size() / 4),
                                   s.prog.data(), s.f.data(), int(s.f.size()), 1, &reg, &vt, &tmp);
      if (rc != MK_OK) return rc;
      if (mode == 1) {
        rc = mk_col_sum(st, vt, i[12], i[13], tmp, static_cast<float*>(P(size_t(n_in))), P(size_t(n_in + 2)));
      } else {
        uint32_t ib = uint32_t(i[15]);
        float init;
        memcpy(&init, &ib, 4);
        rc = mk_row_reduce(st, vt, int(i[10]), int(i[11]), i[12], i[13], tmp, init, P(size_t(n_in)));
      }
      // the stored copy: the value itself (tmp is that buffer) or its bf16 rounding
      if (rc == MK_OK && store && i[16] == 2) rc = mk_convert(st, vt, MK_BF16, i[12] * i[13], tmp, P(size_t(n_in + 3)));
      return rc;
    }
    case StepKind::kGather:
      return mk_gather_rows(st, i[0], i[1], P(0), int(i[2]), i[3], P(1), P(2));
    case StepKind::kScatterAdd:
      return mk_scatter_add_rows(st, int(i[0]), i[1], i[2], P(0), int(i[3]), i[4], P(1), P(2), P(3), P(4));
    case StepKind::kIota:
      return mk_iota(st, int(i[0]), int(i[1]), &i[3], int(i[2]), P(0));
    case StepKind::kCopyStrided:
      return mk_copy_strided(st, int(i[0]), int(i[1]), &i[2], P(0), s.strides.data(), P(1));
    case StepKind::kSoftmax:
      return mk_softmax_rows(st, int(i[0]), i[1], i[2], P(0), P(1));
    case StepKind::kConvert:
      return mk_convert(st, int(i[0]), int(i[1]), i[2], P(0), P(1));
    case StepKind::kFill:
      return mk_fill(st, int(i[0]), i[1], uint64_t(i[2]), P(0));
    case StepKind::kCopy: {
      if (i[0] == 0 || P(0) == P(1)) return MK_OK;  // same memory: an output written over its donated input
      hipError_t e = hipMemcpyAsync(P(1), P(0), size_t(i[0]), hipMemcpyDeviceToDevice, stream);
      if (e == hipSuccess) return MK_OK;
      *f.error = std::string("hipMemcpyAsync: ") + hipGetErrorString(e);
      return MK_ERR_LAUNCH;
    }
  }
  return MK_ERR_UNSUPPORTED;
}

}  // namespace

std::string Run(Program& prog, exec::DeviceContext& dev, const std::vector<RunInput>& inputs,
                std::vector<RunOutput>& outputs, const std::vector<void*>* preset) {
  if (inputs.size() != prog.inputs.size()) return "jam run: wrong number of inputs";  // jam_run.mm:364
  for (size_t k = 0; k < inputs.size(); ++k) {
    if (inputs[k].nbytes != prog.inputs[k].bytes()) return "jam run: input size mismatch";  // jam_run.mm:376
    if (!inputs[k].data && inputs[k].nbytes != 0) return "jam run: null input buffer";
  }
  std::string err;
  std::vector<void*>* consts = prog.DeviceConsts(dev.ordinal());
  if (!consts) return "jam run: constant upload failed";
  if (preset && preset->size() != prog.outputs.size()) return "jam run: preset output list has the wrong length";
  std::vector<RunOutput> outs(prog.outputs.size());
  std::vector<bool> owned(outs.size(), true);
  auto release = [&]() {
    for (size_t k = 0; k < outs.size(); ++k)
      if (owned[k]) dev.Free(outs[k].data);
  };
  for (size_t k = 0; k < outs.size(); ++k) {
    outs[k].type = prog.outputs[k];
    outs[k].nbytes = prog.outputs[k].bytes();
    if (outs[k].nbytes == 0) continue;
    if (preset && (*preset)[k]) {
      outs[k].data = (*preset)[k];
      owned[k] = false;
      continue;
    }
    outs[k].data = dev.Alloc(outs[k].nbytes, &err);
    if (!outs[k].data) {
      release();
      return "jam run: output allocation failed: " + err;
    }
  }
  char* arena = nullptr;
  if (prog.arena_bytes) {
    arena = static_cast<char*>(dev.Alloc(prog.arena_bytes, &err));
    if (!arena) {
      release();
      return "jam run: arena allocation failed: " + err;
    }
  }
  if (!exec::UseDevice(dev.ordinal(), &err)) {
    release();
    dev.Free(arena);
    return "jam run: " + err;
  }
  // generated ew kernels: compiled on the plan's first run, loaded once per
  // device; when that fails the interpreter runs them (reported once)
  void* const* jit_fns = nullptr;
  if (prog.ew_jit) {
    jit_fns = prog.ew_jit->Functions(dev.ordinal());
    if (!jit_fns && prog.ew_jit->strict) {
      release();
      dev.Free(arena);
      return "jam run: generated elementwise kernels unavailable: " + prog.ew_jit->error();
    }
    if (!jit_fns) {
      static std::once_flag warned;
      std::call_once(warned, [&] {
        fprintf(stderr, "jam: generated elementwise kernels unavailable (%s); running the interpreter\n",
                prog.ew_jit->error().c_str());
      });
    }
  }
  std::string step_error;
  Frame f{&inputs, &outs, consts, arena, prog.ew_jit.get(), jit_fns, &step_error};
  for (size_t k = 0; k < prog.steps.size(); ++k) {
    const int rc = RunStep(prog.steps[k], f, dev.stream());
    if (rc != MK_OK) {
      std::string msg = "jam run: step " + std::to_string(k) + " (" + StepName(prog.steps[k].kind) + "): " +
                        (!step_error.empty() ? step_error : std::string(mk_last_error()));
      (void)dev.Synchronize(nullptr);
      release();
      dev.Free(arena);
      return msg;
    }
  }
  // the arena goes back to the pool now: later work on the same stream is
  // ordered after these launches
  dev.Free(arena);
  outputs = std::move(outs);
  return "";
}

}  // namespace mi::jam
