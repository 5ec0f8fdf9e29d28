# FlashMaxSimHIPExt.jl -- weak-dependency extension of FlashMaxSim.jl that
# routes the fused MaxSim forward on AMDGPU.jl arrays (MI355X / gfx950) to
# libflashmaxsim_hip.so through `ccall`.
#
# It specialises exactly the device plugin boundary that the CUDA extension
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
# the device pullbacks on the argmax tape (both strategy markers; the library
# runs the gather + destination-CSR form for either, overwriting the
# zeros_like gradients it is handed):
#   pair_apply_pullback!        src/backward_pair.jl:73-87
#   paired_apply_pullback!      src/backward_layouts.jl:45-60
#   inbatch_apply_pullback!     src/backward_layouts.jl:113-127
#   candidates_apply_pullback!  src/backward_layouts.jl:187-202
#   packed_apply_pullback!      src/packed.jl:384-390
#   varlen_apply_pullback!      src/packed.jl:449-455
# and additionally candidates_forward_ka (src/forward_layouts.jl:272-290), so
# the candidate layout uses the library's fused Σ_t + `neg` epilogue instead
# of the separate `sum(partial; dims=1)` and `ifelse.` kernels.
# Two functions have no reference method and are called through the
# extension module: packed_multi_scan (nq queries against one PackedSeq in
# one pass) and topk (the k best scores of every query column).
#
# Arrays are passed as raw device pointers in Julia's own column-major
# layout, which is the layout the C ABI documents; nothing is copied or
# transposed.  Every call is enqueued on AMDGPU.jl's task-local stream and
# returns without synchronising (src/ka.jl:3-5).  A nonzero status becomes
# an ArgumentError, like the reference's pre-launch checks.
#
# Julia is not installed in the build container, so this file is written to
# the AMDGPU.jl 1.x API and is not exercised by the repository's tests; the
# Python host mirror (flashmaxsim.jl_amd/flashmaxsim) drives the same C ABI
# in the test suite.
module FlashMaxSimHIPExt

using AMDGPU
using FlashMaxSim

const libfms = get(ENV, "FLASHMAXSIM_HIP_LIB",
                   joinpath(@__DIR__, "..", "..", "lib", "libflashmaxsim_hip.so"))

const FMS_F32 = Int32(0)
const FMS_F16 = Int32(1)
const FMS_BF16 = Int32(2)

const ROCBackend = AMDGPU.ROCBackend

@static if isdefined(Core, :BFloat16)
    const FloatFeature = Union{Float16, Float32, Core.BFloat16}
    dtype_code(::Type{Core.BFloat16}) = FMS_BF16
else
    const FloatFeature = Union{Float16, Float32}
end
dtype_code(::Type{Float32}) = FMS_F32
dtype_code(::Type{Float16}) = FMS_F16

stream_ptr() = AMDGPU.stream().stream
dptr(x::ROCArray) = Ptr{Cvoid}(UInt(pointer(x)))
dptr(::Nothing) = C_NULL

function check(status::Int32, what::AbstractString)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:fms_status_string, libfms), Cstring, (Int32,), status))
    throw(ArgumentError("FlashMaxSim HIP $what: $msg"))
end

gfx950() = ccall((:fms_arch_supported, libfms), Cint, ()) == 1

FlashMaxSim.tensor_cores_active(::ROCBackend, ::Type{T}) where {T<:FloatFeature} = gfx950()
FlashMaxSim.tensor_cores_active(::ROCBackend, ::Type{Int8}) = gfx950()

# ---- float scans -------------------------------------------------------------

function FlashMaxSim.launch_pair_scan!(::ROCBackend, argmax_u, partial,
                                       q::ROCMatrix{T}, d::ROCMatrix{T},
                                       qmask, dmask) where {T<:FloatFeature}
    dim, Tq = size(q)
    check(ccall((:fms_launch_pair_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(argmax_u), dptr(partial), dptr(q), dptr(d),
                dptr(qmask), dptr(dmask), dim, Tq, size(d, 2), C_NULL, Int32(0), stream_ptr()),
          "pair scan")
    nothing
end

function FlashMaxSim.launch_paired_scan!(::ROCBackend, args, partial,
                                         Q::ROCArray{T,3}, D::ROCArray{T,3},
                                         qmask, dmask) where {T<:FloatFeature}
    dim, Tq, B = size(Q)
    check(ccall((:fms_launch_paired_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(partial), dptr(Q), dptr(D),
                dptr(qmask), dptr(dmask), dim, Tq, size(D, 2), B, C_NULL, Int32(0), stream_ptr()),
          "paired scan")
    nothing
end

function candidates_call(args, partial, scores, Q::ROCArray{T,3}, gallery, idx,
                         qmask, dmask, N, neg) where {T<:FloatFeature}
    dim, Tq, B = size(Q)
    check(ccall((:fms_launch_candidates_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32,
                 Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64, Int64,
                 Ptr{Cvoid}, Float32, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(partial), dptr(Q), dptr(gallery),
                dptr(idx), Int32(sizeof(eltype(idx))), dptr(qmask), dptr(dmask),
                dim, Tq, B, size(gallery, 2), N, size(idx, 1),
                dptr(scores), Float32(neg), Int32(0), stream_ptr()),
          "candidate scan")
    nothing
end

FlashMaxSim.launch_candidates_scan!(::ROCBackend, args, partial, Q::ROCArray{T,3},
                                    gallery::ROCArray{T,3}, idx, qmask, dmask,
                                    N) where {T<:FloatFeature} =
    candidates_call(args, partial, nothing, Q, gallery, idx, qmask, dmask, N, 0)

# Fused driver: Σ_t and the `neg` fill happen inside the scan kernel
# (replaces src/forward_layouts.jl:285-287).  Same outputs as the reference
# driver: (scores (C,B) in score_eltype(T), args (Tq,C,B)).
function FlashMaxSim.candidates_forward_ka(backend::ROCBackend, Q::ROCArray{T,3},
                                           gallery::ROCArray{T,3},
                                           idxs::AbstractMatrix{<:Integer},
                                           qmask::AbstractMatrix{Bool},
                                           dmask::AbstractMatrix{Bool},
                                           neg::T) where {T<:FloatFeature}
    _, Tq, B, _, N = FlashMaxSim.require_candidates_shapes(Q, gallery, idxs, qmask, dmask)
    idx = FlashMaxSim.indices_on(Q, idxs)
    C = size(idx, 1)
    args = FlashMaxSim.zeros_like(Q, Int32, Tq, C, B)
    S = similar(Q, FlashMaxSim.score_eltype(T), C, B)
    candidates_call(args, nothing, S, Q, gallery, idx, qmask, dmask, N, neg)
    S, args
end

function FlashMaxSim.inbatch_device_scan!(::ROCBackend, S, args,
                                          Q::ROCArray{T,3}, D::ROCArray{T,3},
                                          qmask, dmask) where {T<:FloatFeature}
    dim, Tq, Bq = size(Q)
    check(ccall((:fms_inbatch_device_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(S), dptr(args), dptr(Q), dptr(D),
                dptr(qmask), dptr(dmask), dim, Tq, Bq, size(D, 2), size(D, 3), Int32(0),
                stream_ptr()),
          "in-batch scan")
    nothing
end

function FlashMaxSim.launch_packed_scan!(::ROCBackend, args, partial, q::ROCMatrix{T},
                                         packed::ROCMatrix{T}, cu::ROCVector{Int32},
                                         qmask) where {T<:FloatFeature}
    dim, Tq = size(q)
    check(ccall((:fms_launch_packed_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(partial), dptr(q), dptr(packed), dptr(cu),
                dptr(qmask), dim, Tq, length(cu) - 1, size(packed, 2), C_NULL, Int32(0),
                stream_ptr()),
          "packed scan")
    nothing
end

function FlashMaxSim.launch_varlen_scan!(::ROCBackend, args, partial, Qp::ROCMatrix{T},
                                         Dp::ROCMatrix{T}, cu_q::ROCVector{Int32},
                                         cu_d::ROCVector{Int32}) where {T<:FloatFeature}
    check(ccall((:fms_launch_varlen_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(partial), dptr(Qp), dptr(Dp),
                dptr(cu_q), dptr(cu_d), size(Qp, 1), size(args, 1), size(args, 2),
                size(Qp, 2), size(Dp, 2), C_NULL, Int32(0), stream_ptr()),
          "varlen scan")
    nothing
end

# ---- INT8 scans ----------------------------------------------------------------

function FlashMaxSim.launch_int8_pair_scan!(::ROCBackend, args, partial, qc::ROCMatrix{Int8},
                                            qs::ROCVector{Float32}, dc::ROCMatrix{Int8},
                                            ds::ROCVector{Float32}, qmask, dmask)
    dim, Tq = size(qc)
    check(ccall((:fms_launch_int8_pair_scan, libfms), Int32,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dptr(args), dptr(partial), dptr(qc), dptr(qs), dptr(dc), dptr(ds),
                dptr(qmask), dptr(dmask), dim, Tq, size(dc, 2), C_NULL, Int32(0), stream_ptr()),
          "INT8 pair scan")
    nothing
end

function FlashMaxSim.launch_int8_paired_scan!(::ROCBackend, args, partial,
                                              Qc::ROCArray{Int8,3}, Qs::ROCMatrix{Float32},
                                              Dc::ROCArray{Int8,3}, Ds::ROCMatrix{Float32},
                                              qmask, dmask)
    dim, Tq, B = size(Qc)
    check(ccall((:fms_launch_int8_paired_scan, libfms), Int32,
                (Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Ptr{Cvoid}, Int32, Ptr{Cvoid}),
                dptr(args), dptr(partial), dptr(Qc), dptr(Qs), dptr(Dc), dptr(Ds),
                dptr(qmask), dptr(dmask), dim, Tq, size(Dc, 2), B, C_NULL, Int32(0), stream_ptr()),
          "INT8 paired scan")
    nothing
end


# ---- pullbacks on the argmax tape ----------------------------------------------
# Δ and inv_n arrive in the feature eltype (convert_scores in src/rrule.jl);
# inv_n === nothing passes NULL (all ones).

for M in (FlashMaxSim.AtomicUnified, FlashMaxSim.InvGrid)
    @eval begin
        function FlashMaxSim.pair_apply_pullback!(::$M, ::ROCBackend, dq, dd,
                                                  q::ROCMatrix{T}, d::ROCMatrix{T}, qmask,
                                                  argmax_u, δ, dim, Tq, Td) where {T<:FloatFeature}
            check(ccall((:fms_pair_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dq), dptr(dd), dptr(q), dptr(d), dptr(qmask),
                        dptr(argmax_u), dptr(δ), dim, Tq, Td, stream_ptr()),
                  "pair pullback")
            nothing
        end

        function FlashMaxSim.paired_apply_pullback!(::$M, ::ROCBackend, dQ, dD,
                                                    Q::ROCArray{T,3}, D::ROCArray{T,3}, qmask,
                                                    args, Δ, inv_n, dim, Tq, B,
                                                    Td) where {T<:FloatFeature}
            check(ccall((:fms_paired_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Q), dptr(D), dptr(qmask),
                        dptr(args), dptr(Δ), dptr(inv_n), dim, Tq, Td, B, stream_ptr()),
                  "paired pullback")
            nothing
        end

        function FlashMaxSim.inbatch_apply_pullback!(::$M, ::ROCBackend, dQ, dD,
                                                     Q::ROCArray{T,3}, D::ROCArray{T,3}, qmask,
                                                     args, Δ, inv_n, dim, Tq, Bq, Td,
                                                     Bd) where {T<:FloatFeature}
            check(ccall((:fms_inbatch_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64,
                         Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Q), dptr(D), dptr(qmask),
                        dptr(args), dptr(Δ), dptr(inv_n), dim, Tq, Td, Bq, Bd, stream_ptr()),
                  "in-batch pullback")
            nothing
        end

        function FlashMaxSim.candidates_apply_pullback!(::$M, ::ROCBackend, dQ, dG,
                                                        Q::ROCArray{T,3}, gallery::ROCArray{T,3},
                                                        idx, qmask, args, Δ, inv_n, dim, Tq, B,
                                                        Td, C, N) where {T<:FloatFeature}
            check(ccall((:fms_candidates_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int32,
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dG), dptr(Q), dptr(gallery), dptr(idx),
                        Int32(sizeof(eltype(idx))), dptr(qmask), dptr(args), dptr(Δ),
                        dptr(inv_n), dim, Tq, B, Td, N, C, stream_ptr()),
                  "candidates pullback")
            nothing
        end

        function FlashMaxSim.packed_apply_pullback!(::$M, ::ROCBackend, Δ, q::ROCMatrix{T},
                                                    P::FlashMaxSim.PackedSeq, qmask, args,
                                                    inv_n) where {T<:FloatFeature}
            dq = similar(q)
            dP = similar(P.tokens)
            dim, Tq = size(q)
            check(ccall((:fms_packed_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dq), dptr(dP), dptr(q), dptr(P.tokens), dptr(P.cu),
                        dptr(qmask), dptr(args), dptr(Δ), dptr(inv_n), dim, Tq,
                        length(P.cu) - 1, size(P.tokens, 2), stream_ptr()),
                  "packed pullback")
            dq, dP
        end

        function FlashMaxSim.varlen_apply_pullback!(::$M, ::ROCBackend, Δ,
                                                    Q::FlashMaxSim.PackedSeq,
                                                    D::FlashMaxSim.PackedSeq, args, inv_n)
            T = eltype(Q.tokens)
            dQ = similar(Q.tokens)
            dD = similar(D.tokens)
            check(ccall((:fms_varlen_pullback, libfms), Int32,
                        (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                         Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64,
                         Int64, Int64, Ptr{Cvoid}),
                        dtype_code(T), dptr(dQ), dptr(dD), dptr(Q.tokens), dptr(D.tokens),
                        dptr(Q.cu), dptr(D.cu), dptr(args), dptr(Δ), dptr(inv_n),
                        size(Q.tokens, 1), size(args, 1), size(args, 2), size(Q.tokens, 2),
                        size(D.tokens, 2), stream_ptr()),
                  "varlen pullback")
            dQ, dD
        end
    end
end

# ---- extensions without a reference method -------------------------------------
# Called as FlashMaxSimHIPExt.packed_multi_scan(Q, P) and
# FlashMaxSimHIPExt.topk(S, k) (Base.get_extension(FlashMaxSim, :FlashMaxSimHIPExt)).

"""
    packed_multi_scan(Q::ROCArray{T,3}, P::PackedSeq; qmask = nothing) -> (S, args)

nq queries `Q (dim, Tq, nq)` against every document of `P` in one pass: `S (B, nq)`
Float32 and the 1-based document-local tape `args (Tq, B, nq)`.  Column i equals
`maxsim(Q[:, :, i], P, qmask[:, i]; normalize)` (src/packed.jl:178-210) within the
score tolerance; `normalize` is fused into the scan's score write.
"""
function packed_multi_scan(Q::ROCArray{T,3}, P::FlashMaxSim.PackedSeq;
                           qmask = nothing, normalize::Bool = false) where {T<:FloatFeature}
    dim, Tq, nq = size(Q)
    B = length(P.cu) - 1
    S = AMDGPU.zeros(Float32, B, nq)
    args = AMDGPU.zeros(Int32, Tq, B, nq)
    (nq == 0 || B == 0) && return S, args
    check(ccall((:fms_launch_packed_multi_scan, libfms), Int32,
                (Int32, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
                 Int64, Int64, Int64, Int64, Int64, Int64, Int32, Ptr{Cvoid}),
                dtype_code(T), dptr(args), dptr(S), dptr(Q), dptr(P.tokens), dptr(P.cu),
                qmask === nothing ? C_NULL : dptr(qmask), dim, Tq, nq, B,
                size(P.tokens, 2), P.max_len, Int32(normalize), stream_ptr()),
          "multi-query packed scan")
    S, args
end

"""
    topk(S::ROCMatrix{Float32}, k) -> (vals, idx)

The k best scores of every column of `S` (one column per query): `vals (k, ncols)`
descending, `idx (k, ncols)` 1-based row indices -- `partialsortperm(S[:, i], 1:k;
rev = true)` with a stable sort, for every column in one launch.  1 <= k <= 1024.
"""
function topk(S::ROCMatrix{Float32}, k::Integer)
    n, ncol = size(S)
    vals = AMDGPU.zeros(Float32, k, ncol)
    idx = AMDGPU.zeros(Int32, k, ncol)
    check(ccall((:fms_topk, libfms), Int32,
                (Ptr{Cvoid}, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}),
                dptr(S), ncol, n, k, dptr(vals), dptr(idx), stream_ptr()),
          "topk")
    vals, idx
end

end # module
