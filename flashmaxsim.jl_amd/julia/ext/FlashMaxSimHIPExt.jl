# FlashMaxSimHIPExt.jl -- weak-dependency extension of FlashMaxSim.jl that
# routes the fused MaxSim forward on AMDGPU.jl arrays (MI355X / gfx950) to
# libflashmaxsim_hip.so through `ccall`.
#
# It specialises the device plugin boundary that the CUDA extension
# specialises (ext/FlashMaxSimCUDAExt.jl:57-167 in FlashMaxSim.jl):
#   launch_pair_scan!        src/forward_pair.jl:118-132
#   launch_paired_scan!      src/forward_layouts.jl:126-143
#   launch_candidates_scan!  src/forward_layouts.jl:292-310
#   inbatch_device_scan!     src/forward_layouts.jl:202-203
#   launch_packed_scan!      src/packed.jl:219-234
#   launch_varlen_scan!      src/packed.jl:298-314
#   launch_int8_pair_scan!   src/quant.jl:139-154
#   launch_int8_paired_scan! src/quant.jl:199-217
#   tensor_cores_active      src/ka.jl:71
# the layout drivers that allocate the boundary's buffers, so that every
# float layout uses the library's fused Σ_t / `neg` / tape epilogue:
#   pair_forward_ka          src/forward_pair.jl:104-116
#   paired_forward_ka        src/forward_layouts.jl:112-124
#   inbatch_forward_ka       src/forward_layouts.jl:188-200
#   candidates_forward_ka    src/forward_layouts.jl:272-290
#   packed_forward_ka        src/packed.jl:178-202
#   varlen_forward_ka        src/packed.jl:262-284
# the device quantiser (quantize_int8_symmetric, src/quant.jl:42-49), and the
# device pullbacks on the argmax tape (both strategy markers; the library runs
# the gather + destination-CSR form for either, overwriting the zeros_like
# gradients it is handed):
#   pair_apply_pullback!        src/backward_pair.jl:73-87
#   paired_apply_pullback!      src/backward_layouts.jl:45-60
#   inbatch_apply_pullback!     src/backward_layouts.jl:113-127
#   candidates_apply_pullback!  src/backward_layouts.jl:187-202
#   packed_apply_pullback!      src/packed.jl:384-390
#   varlen_apply_pullback!      src/packed.jl:449-455
# Three functions have no reference method and are called through the
# extension module: packed_multi_scan (nq queries against one PackedSeq in
# one pass), topk (the k best scores of every query column) and
# load_int8_index (an Int8Index read from its at-rest file).
#
# Score buffers.  Every scan entry point writes Float32 partials and scores.
# The reference allocates them as dot_accum(T) / score_eltype(T)
# (src/kernels_forward.jl:16-21): Float32 for Float16 and Float32 features,
# but BFloat16 for BFloat16 features.  So the buffer-taking launch_*! and
# inbatch_device_scan! methods below require Float32 buffers in their
# signatures (a BFloat16 buffer matches none of them and keeps the
# reference's own KA path), and BFloat16 features reach the library only
# through the *_forward_ka drivers, which allocate Float32 outputs
# themselves.  BFloat16 scores therefore come back Float32: the library
# accumulates in fp32 for every 16-bit type, where the reference would
# accumulate BFloat16 in BFloat16.
#
# Arrays are passed as raw device pointers in Julia's own column-major
# layout, which is the layout the C ABI documents; nothing is copied or
# transposed.  Every call is enqueued on AMDGPU.jl's task-local stream and
# returns without synchronising (src/ka.jl:3-5).  A nonzero status becomes
# an ArgumentError, like the reference's pre-launch checks.
#
# Two guards keep every other case on the reference's own path, as the CUDA
# extension does when its tensor cores are off (ext/FlashMaxSimCUDAExt.jl:60-66):
#   - the architecture: each method first asks the library whether the current
#     device is gfx950 (cached per device) and otherwise `@invoke`s the method
#     it overrides (the KernelAbstractions tile kernels, the reference drivers,
#     the reference quantiser and pullbacks);
#   - the array kind: only dense ROCArrays have a pointer the library may read,
#     so masks, indices, inverse counts and PackedSeq storage are typed as
#     dense device arrays in the signatures.  A wrapped array (a
#     PermutedDimsArray, a strided view, src/colocation.jl:18-24) matches none
#     of these methods and dispatch keeps the reference method.
#
# Julia is not installed in the build container, so this file is written to
# the AMDGPU.jl 1.x API and its `ccall`s are checked against the C header by
# a parser in the repository's CPU tests (symbol, arity, argument types and
# argument order, the guards above); the Python host mirror
# (flashmaxsim.jl_amd/flashmaxsim) drives the same C ABI on the GPU.
module FlashMaxSimHIPExt

using AMDGPU
using FlashMaxSim
using FlashMaxSim: PackedSeq, Int8Index

const libfms = joinpath(@__DIR__, "..", "..", "lib", "libflashmaxsim_hip.so")

const FMS_F32 = Int32(0)
const FMS_F16 = Int32(1)
const FMS_BF16 = Int32(2)

const ROCBackend = AMDGPU.ROCBackend
# The backend types the overridden reference methods are declared on.
const KABackend = FlashMaxSim.KernelAbstractions.Backend
const KAGPU = FlashMaxSim.KernelAbstractions.GPU

# Feature types whose reference-allocated partial / score buffers are Float32.
const ScanFeature = Union{Float16, Float32}
# Scale types of an Int8Index whose dot_accum is Float32.
const ScaleType = Union{Float16, Float32}

@static if isdefined(Core, :BFloat16)
    const AnyFeature = Union{Float16, Float32, Core.BFloat16}
    dtype_code(::Type{Core.BFloat16}) = FMS_BF16
else
    const AnyFeature = ScanFeature
end
dtype_code(::Type{Float32}) = FMS_F32
dtype_code(::Type{Float16}) = FMS_F16

# Arguments whose pointer reaches the library: dense device arrays only.
const DenseMask{N} = ROCArray{Bool,N}
const MaybeMask{N} = Union{ROCArray{Bool,N}, Nothing}
# Index eltypes the library reads (4 or 8 bytes; a value outside 1..N is invalid
# under either signedness).
const IndexEltype = Union{Int32, Int64, UInt32, UInt64}
const DenseIndex = ROCMatrix{<:IndexEltype}
const DensePacked{T} = PackedSeq{<:ROCMatrix{T}, <:ROCVector{Int32}}

stream_ptr() = AMDGPU.stream().stream
dptr(x::ROCArray) = Ptr{Cvoid}(UInt(pointer(x)))
dptr(::Nothing) = C_NULL

function check(status::Int32, what::AbstractString)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:fms_status_string, libfms), Cstring, (Int32,), status))
    throw(ArgumentError("FlashMaxSim HIP $what: $msg"))
end

# Whether the current device runs the library's kernels (gfx950).  The library
# caches the answer per device; the ccall itself costs a few nanoseconds.
gfx950() = ccall((:fms_arch_supported, libfms), Cint, ()) == 1

# The extension-only functions have no reference method to fall back to.
require_gfx950(what) = gfx950() ||
    throw(ArgumentError("FlashMaxSim HIP $what: the current device is not gfx950"))

FlashMaxSim.tensor_cores_active(::ROCBackend, ::Type{T}) where {T<:AnyFeature} = gfx950()
FlashMaxSim.tensor_cores_active(::ROCBackend, ::Type{Int8}) = gfx950()

# ---- C entry points (one Julia function per ccall) ------------------------------
# `partial` / `scores` may be `nothing` (NULL): the fused drivers pass scores
# only, the boundary methods partials only.

function c_pair_scan(dtype, argmax_u, partial, q, d, qmask, dmask, dim, Tq, Td, score)
    check(ccall((:fms_launch_pair_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype, dptr(argmax_u), dptr(partial), dptr(q), dptr(d), dptr(qmask),
                dptr(dmask), dim, Tq, Td, dptr(score), Int32(0), stream_ptr()),
          "pair scan")
end

function c_paired_scan(dtype, args, partial, Q, D, qmask, dmask, dim, Tq, Td, B, scores;
                       normalize::Bool = false)
    check(ccall((:fms_launch_paired_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype, dptr(args), dptr(partial), dptr(Q), dptr(D), dptr(qmask), dptr(dmask),
                dim, Tq, Td, B, dptr(scores), Int32(normalize), stream_ptr()),
          "paired scan")
end

function c_candidates_scan(dtype, args, partial, Q, gallery, idx, qmask, dmask,
                           dim, Tq, B, Td, N, C, scores, neg; normalize::Bool = false)
    check(ccall((:fms_launch_candidates_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32,
                 Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64, Int64,
                 Ptr{Cvoid}, Float32, Int32, Ptr{Cvoid}),
                dtype, dptr(args), dptr(partial), dptr(Q), dptr(gallery), dptr(idx),
                Int32(sizeof(eltype(idx))), dptr(qmask), dptr(dmask), dim, Tq, B, Td, N, C,
                dptr(scores), Float32(neg), Int32(normalize), stream_ptr()),
          "candidate scan")
end

# args = nothing: S alone (no tape made; the kernel keeps a running maximum
# without the argmax).  normalize: S .* inv_token_counts(qmask) fused into the
# score write (normalize.jl:18-25).
function c_inbatch_scan(dtype, S, args, Q, D, qmask, dmask, dim, Tq, Bq, Td, Bd;
                        normalize::Bool = false)
    check(ccall((:fms_inbatch_device_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Int32, Ptr{Cvoid}),
                dtype, dptr(S), dptr(args), dptr(Q), dptr(D), dptr(qmask), dptr(dmask),
                dim, Tq, Bq, Td, Bd, Int32(normalize), stream_ptr()),
          "in-batch scan")
end

function c_packed_scan(dtype, args, partial, q, tokens, cu, qmask, dim, Tq, B, ntokens, scores)
    check(ccall((:fms_launch_packed_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype, dptr(args), dptr(partial), dptr(q), dptr(tokens), dptr(cu), dptr(qmask),
                dim, Tq, B, ntokens, dptr(scores), Int32(0), stream_ptr()),
          "packed scan")
end

function c_varlen_scan(dtype, args, partial, Qtokens, Dtokens, cu_q, cu_d, dim, max_q, N,
                       nq_tokens, nd_tokens, scores)
    check(ccall((:fms_launch_varlen_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype, dptr(args), dptr(partial), dptr(Qtokens), dptr(Dtokens), dptr(cu_q),
                dptr(cu_d), dim, max_q, N, nq_tokens, nd_tokens, dptr(scores), Int32(0),
                stream_ptr()),
          "varlen scan")
end

# ---- float scans: the boundary methods (reference-allocated Float32 buffers) ------
# Each falls back to the reference's KernelAbstractions tile kernels
# (`launch_*_scan!(backend::GPU, ...)`, e.g. src/forward_pair.jl:130-132) on any
# other AMD architecture.

function FlashMaxSim.launch_pair_scan!(backend::ROCBackend, argmax_u::ROCVector{Int32},
                                       partial::ROCVector{Float32},
                                       q::ROCMatrix{T}, d::ROCMatrix{T},
                                       qmask::DenseMask{1}, dmask::DenseMask{1}) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.launch_pair_scan!(backend::KAGPU, argmax_u, partial, q, d, qmask, dmask)
    dim, Tq = size(q)
    c_pair_scan(dtype_code(T), argmax_u, partial, q, d, qmask, dmask, dim, Tq, size(d, 2),
                nothing)
    nothing
end

function FlashMaxSim.launch_paired_scan!(backend::ROCBackend, args::ROCMatrix{Int32},
                                         partial::ROCMatrix{Float32},
                                         Q::ROCArray{T,3}, D::ROCArray{T,3},
                                         qmask::DenseMask{2}, dmask::DenseMask{2}) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.launch_paired_scan!(backend::KAGPU, args, partial, Q, D, qmask, dmask)
    dim, Tq, B = size(Q)
    c_paired_scan(dtype_code(T), args, partial, Q, D, qmask, dmask, dim, Tq, size(D, 2), B,
                  nothing)
    nothing
end

function FlashMaxSim.launch_candidates_scan!(backend::ROCBackend, args::ROCArray{Int32,3},
                                             partial::ROCArray{Float32,3},
                                             Q::ROCArray{T,3}, gallery::ROCArray{T,3},
                                             idx::DenseIndex, qmask::DenseMask{2},
                                             dmask::DenseMask{2}, N) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.launch_candidates_scan!(backend::KAGPU, args, partial, Q, gallery, idx, qmask, dmask, N)
    dim, Tq, B = size(Q)
    c_candidates_scan(dtype_code(T), args, partial, Q, gallery, idx, qmask, dmask,
                      dim, Tq, B, size(gallery, 2), N, size(idx, 1), nothing, 0)
    nothing
end

function FlashMaxSim.inbatch_device_scan!(backend::ROCBackend, S::ROCMatrix{Float32},
                                          args::ROCArray{Int32,3},
                                          Q::ROCArray{T,3}, D::ROCArray{T,3},
                                          qmask::DenseMask{2}, dmask::DenseMask{2}) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.inbatch_device_scan!(backend::Any, S, args, Q, D, qmask, dmask)
    dim, Tq, Bq = size(Q)
    c_inbatch_scan(dtype_code(T), S, args, Q, D, qmask, dmask, dim, Tq, Bq, size(D, 2),
                   size(D, 3))
    nothing
end

function FlashMaxSim.launch_packed_scan!(backend::ROCBackend, args::ROCMatrix{Int32},
                                         partial::ROCMatrix{Float32}, q::ROCMatrix{T},
                                         tokens::ROCMatrix{T}, cu::ROCVector{Int32},
                                         qmask::DenseMask{1}) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.launch_packed_scan!(backend::KAGPU, args, partial, q, tokens, cu, qmask)
    dim, Tq = size(q)
    c_packed_scan(dtype_code(T), args, partial, q, tokens, cu, qmask, dim, Tq,
                  length(cu) - 1, size(tokens, 2), nothing)
    nothing
end

function FlashMaxSim.launch_varlen_scan!(backend::ROCBackend, args::ROCMatrix{Int32},
                                         partial::ROCMatrix{Float32}, Qtokens::ROCMatrix{T},
                                         Dtokens::ROCMatrix{T}, cu_q::ROCVector{Int32},
                                         cu_d::ROCVector{Int32}) where {T<:ScanFeature}
    gfx950() || return @invoke FlashMaxSim.launch_varlen_scan!(backend::KAGPU, args, partial, Qtokens, Dtokens, cu_q, cu_d)
    c_varlen_scan(dtype_code(T), args, partial, Qtokens, Dtokens, cu_q, cu_d,
                  size(Qtokens, 1), size(args, 1), size(args, 2), size(Qtokens, 2),
                  size(Dtokens, 2), nothing)
    nothing
end

# ---- float scans: the layout drivers (Float32 outputs allocated here) -----------
# Same results as the reference drivers: (scores, args) with scores in Float32
# (score_eltype(T) for Float16 / Float32 features; Float32 in place of BFloat16
# for BFloat16 features, see the header).  Σ_t and the `neg` fill run inside
# the scan kernel instead of the separate `sum(partial; dims = 1)` and
# `ifelse.` kernels.  On another architecture each invokes the reference
# driver it replaces.

function FlashMaxSim.pair_forward_ka(backend::ROCBackend, q::ROCMatrix{T}, d::ROCMatrix{T},
                                     qmask::DenseMask{1}, dmask::DenseMask{1},
                                     neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.pair_forward_ka(backend::KABackend, q, d, qmask, dmask, neg)
    dim, Tq, Td = FlashMaxSim.require_pair_shapes(q, d, qmask, dmask)
    argmax_u = AMDGPU.zeros(Int32, Tq)
    score = AMDGPU.zeros(Float32, 1)     # length-1, stays on the device
    c_pair_scan(dtype_code(T), argmax_u, nothing, q, d, qmask, dmask, dim, Tq, Td, score)
    score, argmax_u
end

function FlashMaxSim.paired_forward_ka(backend::ROCBackend, Q::ROCArray{T,3}, D::ROCArray{T,3},
                                       qmask::DenseMask{2}, dmask::DenseMask{2},
                                       neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.paired_forward_ka(backend::Any, Q, D, qmask, dmask, neg)
    dim, Tq, Td, B = FlashMaxSim.require_paired_shapes(Q, D, qmask, dmask)
    args = AMDGPU.zeros(Int32, Tq, B)
    scores = AMDGPU.zeros(Float32, B)
    c_paired_scan(dtype_code(T), args, nothing, Q, D, qmask, dmask, dim, Tq, Td, B, scores)
    scores, args
end

function FlashMaxSim.inbatch_forward_ka(backend::ROCBackend, Q::ROCArray{T,3}, D::ROCArray{T,3},
                                        qmask::DenseMask{2}, dmask::DenseMask{2},
                                        neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.inbatch_forward_ka(backend::Any, Q, D, qmask, dmask, neg)
    dim, Tq, Bq, Td, Bd = FlashMaxSim.require_inbatch_shapes(Q, D, qmask, dmask)
    S = AMDGPU.zeros(Float32, Bd, Bq)
    args = AMDGPU.zeros(Int32, Tq, Bd, Bq)
    (Bd == 0 || Bq == 0 || Tq == 0 || Td == 0) && return S, args
    c_inbatch_scan(dtype_code(T), S, args, Q, D, qmask, dmask, dim, Tq, Bq, Td, Bd)
    S, args
end

# ---- the InBatch verb: S without a tape ---------------------------------------
# The reference's maxsim(cfg, Q, D, qmask, dmask, InBatch()) keeps S and drops
# the tape (src/dispatch.jl:121-125, `S, _ = inbatch_forward(...)`); here no tape
# is made.  Same S (Float32, as inbatch_forward_ka above), and with
# cfg.normalize the length normalisation fused into the score write.
# Differentiation is unaffected: the reference's rrule for this call
# (src/rrule.jl:84-99) runs inbatch_forward, which keeps the tape.

function FlashMaxSim.maxsim(cfg::FlashMaxSim.MaxSim{T}, Q::ROCArray{T,3}, D::ROCArray{T,3},
                            qmask::DenseMask{2}, dmask::DenseMask{2},
                            layout::FlashMaxSim.InBatch) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.maxsim(cfg, Q::AbstractArray{T,3}, D::AbstractArray{T,3}, qmask::AbstractMatrix{Bool}, dmask::AbstractMatrix{Bool}, layout)
    FlashMaxSim.require_colocated(Q, D, qmask, dmask)
    dim, Tq, Bq, Td, Bd = FlashMaxSim.require_inbatch_shapes(Q, D, qmask, dmask)
    S = AMDGPU.zeros(Float32, Bd, Bq)
    (Bd == 0 || Bq == 0 || Tq == 0 || Td == 0) && return S
    c_inbatch_scan(dtype_code(T), S, nothing, Q, D, qmask, dmask, dim, Tq, Bq, Td, Bd;
                   normalize = cfg.normalize)
    S
end

# The paired and candidate verbs drop the tape in the reference too
# (src/dispatch.jl:80-85, 160-167): the same scans with no tape buffer, scores
# in Float32, cfg.normalize fused into the score write (invalid candidates keep
# neg, as length_normalize_candidates does).

function FlashMaxSim.maxsim(cfg::FlashMaxSim.MaxSim{T}, Q::ROCArray{T,3}, D::ROCArray{T,3},
                            qmask::DenseMask{2}, dmask::DenseMask{2}) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.maxsim(cfg, Q::AbstractArray{T,3}, D::AbstractArray{T,3}, qmask::AbstractMatrix{Bool}, dmask::AbstractMatrix{Bool})
    FlashMaxSim.require_colocated(Q, D, qmask, dmask)
    dim, Tq, Td, B = FlashMaxSim.require_paired_shapes(Q, D, qmask, dmask)
    scores = AMDGPU.zeros(Float32, B)
    c_paired_scan(dtype_code(T), nothing, nothing, Q, D, qmask, dmask, dim, Tq, Td, B, scores;
                  normalize = cfg.normalize)
    scores
end

function FlashMaxSim.maxsim(cfg::FlashMaxSim.MaxSim{T}, Q::ROCArray{T,3}, gallery::ROCArray{T,3},
                            idxs::DenseIndex, qmask::DenseMask{2},
                            dmask::DenseMask{2}) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.maxsim(cfg, Q::AbstractArray{T,3}, gallery::AbstractArray{T,3}, idxs::AbstractMatrix{<:Integer}, qmask::AbstractMatrix{Bool}, dmask::AbstractMatrix{Bool})
    FlashMaxSim.require_colocated(Q, gallery, qmask, dmask)
    dim, Tq, B, Td, N = FlashMaxSim.require_candidates_shapes(Q, gallery, idxs, qmask, dmask)
    idx = FlashMaxSim.indices_on(Q, idxs)
    C = size(idx, 1)
    scores = AMDGPU.zeros(Float32, C, B)
    c_candidates_scan(dtype_code(T), nothing, nothing, Q, gallery, idx, qmask, dmask,
                      dim, Tq, B, Td, N, C, scores, cfg.neg; normalize = cfg.normalize)
    scores
end

function FlashMaxSim.candidates_forward_ka(backend::ROCBackend, Q::ROCArray{T,3},
                                           gallery::ROCArray{T,3}, idxs::DenseIndex,
                                           qmask::DenseMask{2}, dmask::DenseMask{2},
                                           neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.candidates_forward_ka(backend::Any, Q, gallery, idxs, qmask, dmask, neg)
    dim, Tq, B, Td, N = FlashMaxSim.require_candidates_shapes(Q, gallery, idxs, qmask, dmask)
    idx = FlashMaxSim.indices_on(Q, idxs)
    C = size(idx, 1)
    args = AMDGPU.zeros(Int32, Tq, C, B)
    scores = AMDGPU.zeros(Float32, C, B)
    c_candidates_scan(dtype_code(T), args, nothing, Q, gallery, idx, qmask, dmask,
                      dim, Tq, B, Td, N, C, scores, neg)
    scores, args
end

function FlashMaxSim.packed_forward_ka(backend::ROCBackend, q::ROCMatrix{T}, P::DensePacked{T},
                                       qmask::DenseMask{1}, neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.packed_forward_ka(backend::KABackend, q, P, qmask, neg)
    Tq, B = FlashMaxSim.require_packed_shapes(q, P, qmask)
    tokens, cu = P.tokens, P.cu
    args = AMDGPU.zeros(Int32, Tq, B)
    scores = AMDGPU.zeros(Float32, B)
    c_packed_scan(dtype_code(T), args, nothing, q, tokens, cu, qmask, size(q, 1), Tq, B,
                  size(tokens, 2), scores)
    scores, args
end

function FlashMaxSim.varlen_forward_ka(backend::ROCBackend, Q::DensePacked{T},
                                       D::DensePacked{T}, neg::T) where {T<:AnyFeature}
    gfx950() || return @invoke FlashMaxSim.varlen_forward_ka(backend::KABackend, Q, D, neg)
    N, max_q = FlashMaxSim.require_varlen_shapes(Q, D)
    Qtokens, Dtokens, cu_q, cu_d = Q.tokens, D.tokens, Q.cu, D.cu
    args = AMDGPU.zeros(Int32, max_q, N)
    scores = AMDGPU.zeros(Float32, N)
    c_varlen_scan(dtype_code(T), args, nothing, Qtokens, Dtokens, cu_q, cu_d, size(Qtokens, 1),
                  max_q, N, size(Qtokens, 2), size(Dtokens, 2), scores)
    scores, args
end

# ---- INT8 --------------------------------------------------------------------------
# Scales may be Float16 or Float32 (an Int8Index keeps the eltype of the features it
# was quantised from, src/quant.jl:42-49); the scans widen them to Float32 and
# evaluate (qs * ds) * Float32(acc) (src/kernels_int8.jl:17-25).  Partials are
# dot_accum(eltype(qs)) = Float32 for both.

scale_code(::Type{Float32}) = FMS_F32
scale_code(::Type{Float16}) = FMS_F16

function FlashMaxSim.quantize_int8_symmetric(X::ROCArray{T}) where {T<:ScaleType}
    gfx950() || return @invoke FlashMaxSim.quantize_int8_symmetric(X::AbstractArray{T})
    ndims(X) in (2, 3) || throw(ArgumentError("quantize_int8_symmetric takes (dim, T[, B]) features"))
    dim = size(X, 1)
    codes = similar(X, Int8)
    scales = similar(X, T, size(X)[2:end]...)
    ntok = length(scales)
    ntok == 0 || check(ccall((:fms_int8_quantize, libfms), Int32,
                             (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Ptr{Cvoid}),
                             dtype_code(T), dptr(X), dptr(codes), dptr(scales), dim, ntok,
                             stream_ptr()),
                       "INT8 quantiser")
    Int8Index(codes, scales)
end

function FlashMaxSim.launch_int8_pair_scan!(backend::ROCBackend, args::ROCVector{Int32},
                                            partial::ROCVector{Float32}, qc::ROCMatrix{Int8},
                                            qs::ROCVector{S1}, dc::ROCMatrix{Int8},
                                            ds::ROCVector{S2}, qmask::DenseMask{1},
                                            dmask::DenseMask{1}) where {S1<:ScaleType, S2<:ScaleType}
    gfx950() || return @invoke FlashMaxSim.launch_int8_pair_scan!(backend::KAGPU, args, partial, qc, qs, dc, ds, qmask, dmask)
    dim, Tq = size(qc)
    check(ccall((:fms_launch_int8_pair_scan, libfms), Int32,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32, Ptr{Cvoid}, Ptr{Cvoid},
                 Int32, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}, Int32,
                 Ptr{Cvoid}),
                dptr(args), dptr(partial), dptr(qc), dptr(qs), scale_code(S1), dptr(dc),
                dptr(ds), scale_code(S2), dptr(qmask), dptr(dmask), dim, Tq, size(dc, 2),
                C_NULL, Int32(0), stream_ptr()),
          "INT8 pair scan")
    nothing
end

function FlashMaxSim.launch_int8_paired_scan!(backend::ROCBackend, args::ROCMatrix{Int32},
                                              partial::ROCMatrix{Float32},
                                              Qc::ROCArray{Int8,3}, Qs::ROCMatrix{S1},
                                              Dc::ROCArray{Int8,3}, Ds::ROCMatrix{S2},
                                              qmask::DenseMask{2}, dmask::DenseMask{2}) where {S1<:ScaleType, S2<:ScaleType}
    gfx950() || return @invoke FlashMaxSim.launch_int8_paired_scan!(backend::KAGPU, args, partial, Qc, Qs, Dc, Ds, qmask, dmask)
    dim, Tq, B = size(Qc)
    check(ccall((:fms_launch_int8_paired_scan, libfms), Int32,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32, Ptr{Cvoid}, Ptr{Cvoid},
                 Int32, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32,
                 Ptr{Cvoid}),
                dptr(args), dptr(partial), dptr(Qc), dptr(Qs), scale_code(S1), dptr(Dc),
                dptr(Ds), scale_code(S2), dptr(qmask), dptr(dmask), dim, Tq, size(Dc, 2), B,
                C_NULL, Int32(0), stream_ptr()),
          "INT8 paired scan")
    nothing
end

"""
    int8_candidates_scan(Q::ROCArray{T,3}, D::Int8Index, idxs; qmask, dmask, neg) -> (S, args)

The INT8 candidate layout (no reference method: the candidate conventions of
`maxsim(Q, gallery, idxs)`, src/forward_layouts.jl:272-290, applied to an Int8Index
gallery).  Q is quantised on the fly; `S (C, B)` Float32 with `neg` at invalid
indices, `args (Tq, C, B)`.  gfx950 only (there is no reference method to fall
back to).
"""
function int8_candidates_scan(Q::ROCArray{T,3}, D::Int8Index, idxs::DenseIndex;
                              qmask::MaybeMask{2} = nothing, dmask::MaybeMask{2} = nothing,
                              neg::Real = -1.0f4) where {T<:ScaleType}
    require_gfx950("INT8 candidate scan")
    QQ = FlashMaxSim.quantize_int8_symmetric(Q)
    Qc, Qs, Gc, Gs = QQ.codes, QQ.scales, D.codes, D.scales
    (Gc isa ROCArray{Int8,3} && Gs isa ROCMatrix) ||
        throw(ArgumentError("int8_candidates_scan: the Int8Index must be dense device arrays"))
    dim, Tq, B = size(Qc)
    Td, N = size(Gc, 2), size(Gc, 3)
    size(Gc, 1) == dim || throw(DimensionMismatch("feature dim"))
    size(idxs, 2) == B || throw(DimensionMismatch("idxs"))
    eltype(Gs) <: ScaleType || throw(ArgumentError("Int8Index scales must be Float16 or Float32"))
    idx = FlashMaxSim.indices_on(Qc, idxs)
    C = size(idx, 1)
    args = AMDGPU.zeros(Int32, Tq, C, B)
    scores = AMDGPU.zeros(Float32, C, B)
    check(ccall((:fms_launch_int8_candidates_scan, libfms), Int32,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32, Ptr{Cvoid}, Ptr{Cvoid},
                 Int32, Ptr{Cvoid}, Int32, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64,
                 Int64, Int64, Ptr{Cvoid}, Float32, Int32, Ptr{Cvoid}),
                dptr(args), C_NULL, dptr(Qc), dptr(Qs), scale_code(eltype(Qs)), dptr(Gc),
                dptr(Gs), scale_code(eltype(Gs)), dptr(idx), Int32(sizeof(eltype(idx))),
                dptr(qmask), dptr(dmask), dim, Tq, B, Td, N, C, dptr(scores), Float32(neg),
                Int32(0), stream_ptr()),
          "INT8 candidate scan")
    scores, args
end

# ---- pullbacks on the argmax tape ----------------------------------------------
# Δ and inv_n arrive in the feature eltype (convert_scores in src/rrule.jl), and the
# gradients are feature-eltype buffers, which is what the library reads and writes
# for every feature type; inv_n === nothing passes NULL (all ones).  On another
# architecture each invokes the reference method for the same strategy marker.

for M in (FlashMaxSim.AtomicUnified, FlashMaxSim.InvGrid)
    @eval begin
        function FlashMaxSim.pair_apply_pullback!(mode::$M, backend::ROCBackend, dq::ROCMatrix{T},
                                                  dd::ROCMatrix{T}, q::ROCMatrix{T},
                                                  d::ROCMatrix{T}, qmask::MaybeMask{1},
                                                  argmax_u::ROCVector{Int32},
                                                  delta::ROCVector{T}, dim, Tq,
                                                  Td) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.pair_apply_pullback!(mode, backend::Any, dq, dd, q, d, qmask, argmax_u, delta, dim, Tq, Td)
            check(ccall((:fms_pair_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dq), dptr(dd), dptr(q), dptr(d), dptr(qmask),
                        dptr(argmax_u), dptr(delta), dim, Tq, Td, stream_ptr()),
                  "pair pullback")
            nothing
        end

        function FlashMaxSim.paired_apply_pullback!(mode::$M, backend::ROCBackend, dQ::ROCArray{T,3},
                                                    dD::ROCArray{T,3}, Q::ROCArray{T,3},
                                                    D::ROCArray{T,3}, qmask::MaybeMask{2},
                                                    args::ROCMatrix{Int32}, Delta::ROCVector{T},
                                                    inv_n::Union{ROCVector{T}, Nothing}, dim, Tq, B,
                                                    Td) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.paired_apply_pullback!(mode, backend::Any, dQ, dD, Q, D, qmask, args, Delta, inv_n, dim, Tq, B, Td)
            check(ccall((:fms_paired_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Q), dptr(D), dptr(qmask),
                        dptr(args), dptr(Delta), dptr(inv_n), dim, Tq, Td, B, stream_ptr()),
                  "paired pullback")
            nothing
        end

        function FlashMaxSim.inbatch_apply_pullback!(mode::$M, backend::ROCBackend, dQ::ROCArray{T,3},
                                                     dD::ROCArray{T,3}, Q::ROCArray{T,3},
                                                     D::ROCArray{T,3}, qmask::MaybeMask{2},
                                                     args::ROCArray{Int32,3},
                                                     Delta::ROCMatrix{T},
                                                     inv_n::Union{ROCVector{T}, Nothing}, dim, Tq, Bq,
                                                     Td, Bd) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.inbatch_apply_pullback!(mode, backend::Any, dQ, dD, Q, D, qmask, args, Delta, inv_n, dim, Tq, Bq, Td, Bd)
            check(ccall((:fms_inbatch_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64,
                         Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Q), dptr(D), dptr(qmask),
                        dptr(args), dptr(Delta), dptr(inv_n), dim, Tq, Td, Bq, Bd, stream_ptr()),
                  "in-batch pullback")
            nothing
        end

        function FlashMaxSim.candidates_apply_pullback!(mode::$M, backend::ROCBackend, dQ::ROCArray{T,3},
                                                        dG::ROCArray{T,3}, Q::ROCArray{T,3},
                                                        gallery::ROCArray{T,3}, idx::DenseIndex,
                                                        qmask::MaybeMask{2},
                                                        args::ROCArray{Int32,3},
                                                        Delta::ROCMatrix{T},
                                                        inv_n::Union{ROCVector{T}, Nothing}, dim, Tq, B,
                                                        Td, C, N) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.candidates_apply_pullback!(mode, backend::Any, dQ, dG, Q, gallery, idx, qmask, args, Delta, inv_n, dim, Tq, B, Td, C, N)
            check(ccall((:fms_candidates_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32,
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dG), dptr(Q), dptr(gallery), dptr(idx),
                        Int32(sizeof(eltype(idx))), dptr(qmask), dptr(args), dptr(Delta),
                        dptr(inv_n), dim, Tq, B, Td, N, C, stream_ptr()),
                  "candidates pullback")
            nothing
        end

        function FlashMaxSim.packed_apply_pullback!(mode::$M, backend::ROCBackend, Delta::ROCVector{T},
                                                    q::ROCMatrix{T}, P::DensePacked{T},
                                                    qmask::MaybeMask{1}, args::ROCMatrix{Int32},
                                                    inv_n::Union{ROCVector{T}, Nothing}) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.packed_apply_pullback!(mode, backend::Any, Delta, q, P, qmask, args, inv_n)
            tokens, cu = P.tokens, P.cu
            dq = similar(q)
            dP = similar(tokens)
            dim, Tq = size(q)
            check(ccall((:fms_packed_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dq), dptr(dP), dptr(q), dptr(tokens), dptr(cu),
                        dptr(qmask), dptr(args), dptr(Delta), dptr(inv_n), dim, Tq,
                        length(cu) - 1, size(tokens, 2), stream_ptr()),
                  "packed pullback")
            dq, dP
        end

        function FlashMaxSim.varlen_apply_pullback!(mode::$M, backend::ROCBackend, Delta::ROCVector{T},
                                                    Q::DensePacked{T}, D::DensePacked{T},
                                                    args::ROCMatrix{Int32},
                                                    inv_n::Union{ROCVector{T}, Nothing}) where {T<:AnyFeature}
            gfx950() || return @invoke FlashMaxSim.varlen_apply_pullback!(mode, backend::Any, Delta, Q, D, args, inv_n)
            Qtokens, Dtokens, cu_q, cu_d = Q.tokens, D.tokens, Q.cu, D.cu
            dQ = similar(Qtokens)
            dD = similar(Dtokens)
            check(ccall((:fms_varlen_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Qtokens), dptr(Dtokens),
                        dptr(cu_q), dptr(cu_d), dptr(args), dptr(Delta), dptr(inv_n),
                        size(Qtokens, 1), size(args, 1), size(args, 2), size(Qtokens, 2),
                        size(Dtokens, 2), stream_ptr()),
                  "varlen pullback")
            dQ, dD
        end
    end
end

# ---- extensions without a reference method -------------------------------------
# Called as FlashMaxSimHIPExt.packed_multi_scan(Q, P), FlashMaxSimHIPExt.topk(S, k) and
# FlashMaxSimHIPExt.load_int8_index(path)
# (Base.get_extension(FlashMaxSim, :FlashMaxSimHIPExt)).  The first two run on
# gfx950 only and say so otherwise.

"""
    packed_multi_scan(Q::ROCArray{T,3}, P::PackedSeq; qmask = nothing) -> (S, args)

nq queries `Q (dim, Tq, nq)` against every document of `P` in one pass: `S (B, nq)`
Float32 and the 1-based document-local tape `args (Tq, B, nq)`.  Column i equals
`maxsim(Q[:, :, i], P, qmask[:, i]; normalize)` (src/packed.jl:178-210) within the
score tolerance; `normalize` is fused into the scan's score write.
"""
function packed_multi_scan(Q::ROCArray{T,3}, P::DensePacked{T};
                           qmask::MaybeMask{2} = nothing, normalize::Bool = false) where {T<:AnyFeature}
    require_gfx950("multi-query packed scan")
    dim, Tq, nq = size(Q)
    tokens, cu, max_len = P.tokens, P.cu, P.max_len
    B = length(cu) - 1
    scores = AMDGPU.zeros(Float32, B, nq)
    args = AMDGPU.zeros(Int32, Tq, B, nq)
    (nq == 0 || B == 0) && return scores, args
    check(ccall((:fms_launch_packed_multi_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Int64, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(scores), dptr(Q), dptr(tokens), dptr(cu),
                dptr(qmask), dim, Tq, nq, B, size(tokens, 2), max_len, Int32(normalize),
                stream_ptr()),
          "multi-query packed scan")
    scores, args
end

"""
    topk(S::ROCMatrix{Float32}, k) -> (vals, idx)

The k best scores of every column of `S` (one column per query): `vals (k, ncols)`
descending, `idx (k, ncols)` 1-based row indices -- `partialsortperm(S[:, i], 1:k;
rev = true)` with a stable sort, for every column in one launch.  1 <= k <= 1024.
"""
function topk(scores::ROCMatrix{Float32}, k::Integer)
    require_gfx950("topk")
    ncols, nrows = size(scores)   # C rows: one score row per query column
    vals = AMDGPU.zeros(Float32, k, nrows)
    idx = AMDGPU.zeros(Int32, k, nrows)
    check(ccall((:fms_topk, libfms), Int32,
                (Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}),
                dptr(scores), nrows, ncols, k, dptr(vals), dptr(idx), stream_ptr()),
          "topk")
    vals, idx
end

# ---- Int8Index at rest -------------------------------------------------------------
# The file is safetensors: a little-endian UInt64 header length n, n bytes of JSON,
# then the tensor bytes.  The JSON names two tensors, "codes" (dtype "I8", shape
# [N, Td, dim], i.e. Julia's column-major (dim, Td, N)) and "scales" ("F32" or
# "F16", shape [N, Td] = Julia (Td, N)), each with "data_offsets" [begin, end)
# relative to the end of the header, and "__metadata__" with
# "format": "flashmaxsim-int8-index-v1".  The index is read with `read!` into
# host arrays of the reversed shape, byte for byte, with no JSON package: the
# patterns below pick the fields out of the header.

const ST_FORMAT = r"\"format\"\s*:\s*\"flashmaxsim-int8-index-v1\""
const ST_ENTRY_CODES = r"\"codes\"\s*:\s*\{([^}]*)\}"
const ST_ENTRY_SCALES = r"\"scales\"\s*:\s*\{([^}]*)\}"
const ST_DTYPE = r"\"dtype\"\s*:\s*\"([A-Z0-9]+)\""
const ST_SHAPE = r"\"shape\"\s*:\s*\[([0-9,\s]*)\]"
const ST_OFFSETS = r"\"data_offsets\"\s*:\s*\[\s*([0-9]+)\s*,\s*([0-9]+)\s*\]"

const ST_TYPES = Dict("I8" => Int8, "F32" => Float32, "F16" => Float16)

function st_tensor(io::IO, header::AbstractString, data0::Integer, entry::Regex)
    m = match(entry, header)
    m === nothing && throw(ArgumentError("Int8Index file: tensor missing"))
    body = m.captures[1]
    md, ms, mo = match(ST_DTYPE, body), match(ST_SHAPE, body), match(ST_OFFSETS, body)
    (md === nothing || ms === nothing || mo === nothing) &&
        throw(ArgumentError("Int8Index file: malformed tensor entry"))
    T = get(ST_TYPES, md.captures[1]) do
        throw(ArgumentError("Int8Index file: unsupported dtype $(md.captures[1])"))
    end
    shape = [parse(Int, s) for s in split(ms.captures[1], ',') if !isempty(strip(s))]
    b, e = parse(Int, mo.captures[1]), parse(Int, mo.captures[2])
    x = Array{T}(undef, reverse(shape)...)
    e - b == sizeof(x) || throw(ArgumentError("Int8Index file: tensor byte count"))
    seek(io, data0 + b)
    read!(io, x)
    ENDIAN_BOM == 0x04030201 || (x .= ltoh.(x))
    x
end

"""
    load_int8_index(path; device = true) -> Int8Index

Read an Int8Index written by the Python host's `save_int8_index` (the
safetensors layout described above): `codes (dim, Td, N)` Int8 and
`scales (Td, N)` Float32 or Float16, moved to the GPU when `device`.
"""
function load_int8_index(path::AbstractString; device::Bool = true)
    codes, scales = open(path, "r") do io
        n = Int(ltoh(read(io, UInt64)))
        header = String(read(io, n))
        occursin(ST_FORMAT, header) ||
            throw(ArgumentError("$path: not a flashmaxsim-int8-index-v1 file"))
        data0 = 8 + n
        st_tensor(io, header, data0, ST_ENTRY_CODES), st_tensor(io, header, data0, ST_ENTRY_SCALES)
    end
    eltype(codes) === Int8 || throw(ArgumentError("$path: codes must be Int8"))
    eltype(scales) <: ScaleType || throw(ArgumentError("$path: scales must be Float32 or Float16"))
    size(codes)[2:end] == size(scales) || throw(DimensionMismatch("Int8Index token count"))
    device ? Int8Index(ROCArray(codes), ROCArray(scales)) : Int8Index(codes, scales)
end

end # module
