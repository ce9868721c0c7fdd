// Smx.cs -- P/Invoke binding of libsmx.so (include/smx.h) for SmallMind (C#/.NET).
// Not compiled in this repository (no .NET toolchain); tests/test_bindings.py checks every
// declaration below against include/smx.h (names, parameter counts and type mapping).
// The backend classes follow the reference's interfaces: IWeightTensor
// (src/SmallMind.Quantization/Abstractions/IWeightTensor.cs:7-42), TransformerModel.Forward with the
// KV cache (TransformerModel.cs:272-344, ResetKVCache :476-506), InferenceSession's sampling
// options (ProductionInferenceOptions.cs:19-87).
using System;
using System.Collections.Generic;
using System.Diagnostics;
using System.Runtime.InteropServices;
using System.Threading;
using SmallMind.Core.Exceptions;
using SmallMind.Quantization.Abstractions;
using SmallMind.Runtime.Cache;
using SmallMind.Runtime.Execution;

namespace SmallMind.Backends.Rocm
{
    internal static unsafe class Smx
    {
        const string Lib = "smx";   // resolves libsmx.so

        public const int OK = 0, EINVAL = -1, ENOMEM = -2, EDEVICE = -3, EBUSY = -4,
                         EUNSUPPORTED = -5, ESTATE = -6, ERANGE = -7, ECANCELED = -8, ETIMEDOUT = -9;
        public const int F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14;
        // SMQ Q8Tensor / Q4Tensor blocks in their upload layout (smx_smq_pack)
        public const int SMQ_Q8 = 1010, SMQ_Q4 = 1011;

        [StructLayout(LayoutKind.Sequential)]
        public struct ModelConfig            // smx_model_config; ModelConfig.cs:142-258
        {
            public int Arch, Vocab, Ctx, DModel, NLayer, NHead, NKvHead, DFf;
            public float RopeTheta, NormEps;
            public fixed int Reserved[6];
        }

        [StructLayout(LayoutKind.Sequential)]
        public struct GenStats { public double PrefillMs, DecodeMs; public int NPrefill, NDecode; }

        [StructLayout(LayoutKind.Sequential)]
        public struct Sampling               // smx_sampling; ProductionInferenceOptions.cs:19-87
        {
            public float Temperature; public int TopK; public double TopP; public float MinP,
                RepetitionPenalty, PresencePenalty, FrequencyPenalty; public int RepetitionWindow;
        }

        // library and block formats
        [DllImport(Lib)] public static extern IntPtr smx_version();
        [DllImport(Lib)] public static extern IntPtr smx_last_error();
        [DllImport(Lib)] public static extern int smx_type_block_elems(int type);
        [DllImport(Lib)] public static extern int smx_type_block_bytes(int type);
        [DllImport(Lib)] public static extern long smx_type_row_bytes(int type, long k);
        [DllImport(Lib)] public static extern int smx_dequant(int type, void* blocksDev, long n, float* outDev, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_quantize(int type, float* xDev, long n, void* blocksDev, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_fill_normal(ulong seed, long n, float std, float* outDev, IntPtr stream);

        // weights (IWeightTensor)
        [DllImport(Lib)] public static extern int smx_weight_create(int type, long rows, long cols, void* blocks,
            int blocksOnDevice, out IntPtr w);
        [DllImport(Lib)] public static extern int smx_weight_info(IntPtr w, out int type, out long rows, out long cols);
        [DllImport(Lib)] public static extern int smx_weight_matmul(IntPtr w, float* actDev, float* outDev, int m,
            int k, int n, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_weight_matmul_host(IntPtr w, float* act, float* output, int m,
            int k, int n);
        [DllImport(Lib)] public static extern int smx_weight_to_float32_host(IntPtr w, float* output);
        [DllImport(Lib)] public static extern int smx_weight_matmul_noalloc(IntPtr w, float* actDev, float* outDev,
            int m, int k, int n, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_weight_to_float32(IntPtr w, float* outDev, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_weight_destroy(IntPtr w);

        // operators
        [DllImport(Lib)] public static extern int smx_rmsnorm(float* xDev, float* gammaDev, float* yDev, int rows, int n,
            float eps, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_layernorm(float* xDev, float* gammaDev, float* betaDev, float* yDev,
            int rows, int n, float eps, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_rope_tables(int maxPos, int headDim, float theta, float* cosHost,
            float* sinHost);
        [DllImport(Lib)] public static extern int smx_rope(float* dataDev, int nHeads, int seq, int headDim, int pos0,
            float* cosDev, float* sinDev, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_scale_mask_softmax(float* scoresDev, float scale, int seq,
            int kSeq, int cacheOffset, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_attention_decode(float* qDev, float* kCacheDev, float* vCacheDev,
            float* outDev, int nHead, int nKvHead, int headDim, int ctxStride, int nPos, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_attention_prefill(float* qDev, float* kCacheDev, float* vCacheDev,
            float* outDev, int nHead, int nKvHead, int headDim, int ctxStride, int pFirst, int nTok, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_silu_mul(float* gateDev, float* upDev, float* yDev, long n, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_gelu(float* xDev, float* yDev, long n, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_argmax(float* xDev, int n, int* outDev, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_stream_read(void* srcDev, ulong bytes, IntPtr stream);
        [DllImport(Lib)] public static extern int smx_sample(float* logitsDev, int n, int* contextDev, int nContext,
            in Sampling p, double u, float* probsDev, int* tokenDev, IntPtr stream);

        // model and sessions
        [DllImport(Lib)] public static extern int smx_context_create(int device, out IntPtr ctx);
        [DllImport(Lib)] public static extern int smx_context_destroy(IntPtr ctx);
        [DllImport(Lib)] public static extern int smx_model_create(IntPtr ctx, in ModelConfig cfg, out IntPtr model);
        [DllImport(Lib)] public static extern int smx_model_upload_tensor(IntPtr model,
            [MarshalAs(UnmanagedType.LPUTF8Str)] string name, int ggmlType, long* dims, int ndims, void* bytes,
            nuint nbytes, int bytesOnDevice);
        [DllImport(Lib)] public static extern int smx_model_finalize(IntPtr model);
        [DllImport(Lib)] public static extern int smx_model_load_gguf(IntPtr ctx,
            [MarshalAs(UnmanagedType.LPUTF8Str)] string path, out IntPtr model);
        [DllImport(Lib)] public static extern int smx_gguf_read_config([MarshalAs(UnmanagedType.LPUTF8Str)] string path,
            out ModelConfig cfg, out long nTensors);
        // cfg: the ModelConfig argument of SmqModelLoader.LoadFromSmq, or null for the file's metadata
        [DllImport(Lib)] public static extern int smx_model_load_smq(IntPtr ctx,
            [MarshalAs(UnmanagedType.LPUTF8Str)] string path, ModelConfig* cfg, out IntPtr model);
        [DllImport(Lib)] public static extern int smx_smq_read_config([MarshalAs(UnmanagedType.LPUTF8Str)] string path,
            out ModelConfig cfg, out long nTensors);
        [DllImport(Lib)] public static extern int smx_smq_pack(int type, void* data, float* scales, long rows, long cols,
            int blockSize, void* output, nuint outBytes);
        [DllImport(Lib)] public static extern int smx_model_weight_bytes(IntPtr model, out long bytes);
        [DllImport(Lib)] public static extern int smx_model_destroy(IntPtr model);
        [DllImport(Lib)] public static extern int smx_session_create(IntPtr model, int maxCtx, out IntPtr session);
        [DllImport(Lib)] public static extern int smx_session_forward(IntPtr session, int* tokens, int nTokens,
            int posOffset, float* logitsOut);
        [DllImport(Lib)] public static extern int smx_session_generate(IntPtr session, int* prompt, int nPrompt, int nNew,
            int* outTokens, float* logitsOut, GenStats* stats);
        // callable from any thread while another thread is inside a generate call on the session
        [DllImport(Lib)] public static extern int smx_session_cancel(IntPtr session);
        [DllImport(Lib)] public static extern int smx_session_set_max_time(IntPtr session, int maxTimeMs);
        [DllImport(Lib)] public static extern int smx_session_generate_sampled(IntPtr session, int* prompt,
            int nPrompt, int nNew, in Sampling p, ulong seed, int* outTokens, float* logitsOut, GenStats* stats);
        [DllImport(Lib)] public static extern int smx_batch_generate(IntPtr* sessions, int nSessions, int* prompts,
            int* promptLens, int nNew, int* outTokens, GenStats* stats);
        [DllImport(Lib)] public static extern int smx_batcher_create(IntPtr model, int maxMembers, int maxCtx,
            out IntPtr batcher);
        [DllImport(Lib)] public static extern int smx_batcher_add(IntPtr batcher, IntPtr session, int* prompt,
            int nPrompt);
        [DllImport(Lib)] public static extern int smx_batcher_add_sampled(IntPtr batcher, IntPtr session,
            int* prompt, int nPrompt, in Sampling p, ulong seed);
        [DllImport(Lib)] public static extern int smx_batcher_remove(IntPtr batcher, IntPtr session);
        [DllImport(Lib)] public static extern int smx_batcher_count(IntPtr batcher);
        [DllImport(Lib)] public static extern int smx_batcher_step(IntPtr batcher, int nSteps, int* outTokens);
        [DllImport(Lib)] public static extern int smx_batcher_destroy(IntPtr batcher);
        [DllImport(Lib)] public static extern int smx_session_reset(IntPtr session);
        [DllImport(Lib)] public static extern int smx_session_destroy(IntPtr session);

        // Status -> the exception the reference throws at the same point.  maxTimeMs is the
        // session's time limit, reported by InferenceTimeoutException (InferenceSession.cs:287-291).
        public static void Check(int rc, int maxTimeMs = 0)
        {
            if (rc == OK) return;
            string msg = Marshal.PtrToStringUTF8(smx_last_error()) ?? "libsmx error";
            throw rc switch
            {
                EINVAL => new ArgumentException(msg),            // Q8WeightTensor.cs:43-48
                ERANGE => new ArgumentOutOfRangeException(msg),  // TransformerModel.cs:282-285
                EBUSY => new InvalidOperationException(msg),     // InferenceSession.cs:127-144
                ECANCELED => new OperationCanceledException(msg),   // InferenceSession.cs:211, :481
                ETIMEDOUT => new InferenceTimeoutException(maxTimeMs, msg),   // InferenceSession.cs:287-291
                _ => new InvalidOperationException(msg),
            };
        }
    }

    // IWeightTensor (IWeightTensor.cs:7-42) on the device, injected through
    // Linear.SetQuantizedWeight (NeuralNet.cs:84-107).  That injection checks
    // Rows == outFeatures and Cols == inFeatures (NeuralNet.cs:89), and Linear.ForwardQuantized then
    // calls MatMul(input, output, m, k: inFeatures, n: outFeatures) (NeuralNet.cs:168-173, :211-216),
    // so this tensor reports Rows = output features, Cols = input features and accepts
    // k == Cols, n == Rows.  (IWeightTensor.cs:31-32 documents k == Rows and n == Cols, which the
    // reference's own Q8WeightTensor checks (Q8WeightTensor.cs:43-44); for a non-square layer the two
    // reference checks cannot both hold, and this class follows the one Linear enforces.)  The device
    // matrix holds the GGUF [out][in] rows, and the library computes
    // output[m][n] = activations[m][k] . W[n][k]^T.  ToFloat32 returns Rows x Cols = [out][in].
    // Operands stay in host memory; libsmx.so stages them on the device itself (kept per weight, so
    // repeated calls allocate nothing).
    internal sealed unsafe class GpuWeightTensor : IWeightTensor, IDisposable
    {
        readonly IntPtr _w;
        readonly int _in, _out;

        public GpuWeightTensor(int ggmlType, int outFeatures, int inFeatures, ReadOnlySpan<byte> ggufBlocks,
                               QuantScheme scheme)
        {
            _in = inFeatures;
            _out = outFeatures;
            Scheme = scheme;
            fixed (byte* p = ggufBlocks)
                Smx.Check(Smx.smx_weight_create(ggmlType, outFeatures, inFeatures, p, 0, out _w));
        }

        public int Rows => _out;
        public int Cols => _in;
        public QuantScheme Scheme { get; }

        public void MatMul(ReadOnlySpan<float> activations, Span<float> output, int m, int k, int n)
        {
            if (k != Cols) throw new ArgumentException($"k={k} must equal Cols={Cols} (input features)");
            if (n != Rows) throw new ArgumentException($"n={n} must equal Rows={Rows} (output features)");
            if (activations.Length < m * k)
                throw new ArgumentException($"activations.Length {activations.Length} < m*k {m * k}");
            if (output.Length < m * n) throw new ArgumentException($"output.Length {output.Length} < m*n {m * n}");
            fixed (float* a = activations)
            fixed (float* o = output)
                Smx.Check(Smx.smx_weight_matmul_host(_w, a, o, m, k, n));   // output fully overwritten
        }

        public float[] ToFloat32()
        {
            var r = new float[_out * _in];   // [Rows = out][Cols = in], bit-identical to GgufModelLoader's dequantization
            fixed (float* o = r)
                Smx.Check(Smx.smx_weight_to_float32_host(_w, o));
            return r;
        }

        public void Dispose() => Smx.smx_weight_destroy(_w);
    }

    // IRuntimeExecutor (Execution/IRuntimeExecutor.cs:8-27) on the device, in place of
    // RuntimeExecutor (RuntimeExecutor.cs:13-178).  Compiled into SmallMind.Runtime, whose internal
    // types it implements and constructs.  Prefill follows RuntimeExecutor.Prefill step by step: the
    // same argument and state checks, the prompt cropped to its last blockSize tokens (:55-57), the
    // forward at position 0, a KvCacheHandle rented from the pool and stored in the context,
    // context.CurrentPosition = the processed length, and PrefillMetrics from a stopwatch.  The KV
    // cache itself is a device session (smx_session) keyed to that handle: the rented entry is a
    // zero-layer placeholder (ModelShape(0, heads, headDim)), so it holds no host K/V arrays.
    // Decode reads context.CurrentPosition, runs one token on the handle's session and advances the
    // position, as RuntimeExecutor.Decode does (:117-176).
    internal sealed unsafe class GpuRuntimeExecutor : IRuntimeExecutor, IDisposable
    {
        readonly GpuTransformerBackend _backend;
        readonly KvCachePool _cachePool;
        readonly int _blockSize, _vocab, _heads, _headDim;
        readonly Dictionary<KvCacheHandle, GpuSession> _sessions = new(ReferenceEqualityComparer.Instance);

        public GpuRuntimeExecutor(GpuTransformerBackend backend, KvCachePool cachePool, int blockSize, int vocabSize,
                                  int numHeads, int headDim)
        {
            _backend = backend ?? throw new ArgumentNullException(nameof(backend));
            _cachePool = cachePool ?? throw new ArgumentNullException(nameof(cachePool));
            _blockSize = blockSize;
            _vocab = vocabSize;
            _heads = numHeads;
            _headDim = headDim;
        }

        public PrefillResult Prefill(ReadOnlySpan<int> promptTokens, ExecutionContext context)
        {
            if (context == null) throw new ArgumentNullException(nameof(context));
            if (promptTokens.Length == 0)
                throw new ArgumentException("Prompt tokens cannot be empty", nameof(promptTokens));
            if (context.HasCache)
                throw new InvalidOperationException("Context already has a cache. Call Reset() before prefill.");
            var sw = Stopwatch.StartNew();
            int startIdx = Math.Max(0, promptTokens.Length - _blockSize);
            int promptLength = promptTokens.Length - startIdx;
            var promptSlice = promptTokens.Slice(startIdx, promptLength);

            var entry = _cachePool.Rent(new ModelShape(0, _heads, _headDim), _blockSize,
                                        new SessionId(Guid.NewGuid().ToString()));
            var handle = new KvCacheHandle(entry);
            var session = _backend.CreateSession(_blockSize);
            var lastLogits = new float[_vocab];
            try
            {
                session.ForwardLastRow(promptSlice, 0, lastLogits);   // ResetKVCache + Forward(pos 0)
            }
            catch
            {
                session.Dispose();
                _cachePool.Return(entry);
                throw;
            }
            _sessions[handle] = session;
            context.CacheHandle = handle;
            context.CurrentPosition = promptLength;
            sw.Stop();
            var metrics = new PrefillMetrics(promptLength, sw.Elapsed.TotalMilliseconds);
            if (context.Options.EnableTelemetry)
                context.Telemetry.RecordPrefillEnd(promptLength, sw.Elapsed.TotalMilliseconds);
            return new PrefillResult(new ReadOnlyMemory<float>(lastLogits), handle, promptLength, metrics);
        }

        public DecodeResult Decode(int nextToken, ExecutionContext context)
        {
            if (context == null) throw new ArgumentNullException(nameof(context));
            if (!context.HasCache)
            {
                if (context.Options.RequireKvCache)
                    throw new InvalidOperationException(
                        "Context does not have a cache. Call Prefill() first or disable RequireKvCache.");
                throw new InvalidOperationException("Decode requires prefill to be called first");
            }
            if (!_sessions.TryGetValue(context.CacheHandle!, out var session))
                throw new InvalidOperationException("The context's cache was not created by this executor");
            var sw = Stopwatch.StartNew();
            var decodedLogits = new float[_vocab];
            Span<int> t = stackalloc int[1] { nextToken };
            session.ForwardLastRow(t, context.CurrentPosition, decodedLogits);   // Forward(pos = CurrentPosition)
            context.CurrentPosition++;
            sw.Stop();
            var metrics = new DecodeMetrics(sw.Elapsed.TotalMilliseconds, context.CurrentPosition, cacheUsed: true);
            if (context.Options.EnableTelemetry)
                context.Telemetry.RecordDecodeEnd(sw.Elapsed.TotalMilliseconds);
            return new DecodeResult(new ReadOnlyMemory<float>(decodedLogits), context.CacheHandle!, metrics);
        }

        // Releases the device session of a context's cache (the context is then Reset or disposed).
        public void Release(ExecutionContext context)
        {
            if (context?.CacheHandle is KvCacheHandle h && _sessions.Remove(h, out var session))
            {
                session.Dispose();
                _cachePool.Return(h.CacheEntry);
            }
        }

        public void Dispose()
        {
            foreach (var kv in _sessions)
            {
                kv.Value.Dispose();
                _cachePool.Return(kv.Key.CacheEntry);
            }
            _sessions.Clear();
        }
    }

    // The model on the device: loaded from a GGUF or .smq file in one call, or tensor by tensor.
    internal sealed unsafe class GpuTransformerBackend : IDisposable
    {
        readonly IntPtr _ctx, _model;

        public GpuTransformerBackend(string ggufPath, int device = 0)
        {
            Smx.Check(Smx.smx_context_create(device, out _ctx));
            int rc = Smx.smx_model_load_gguf(_ctx, ggufPath, out _model);
            if (rc != 0) { Smx.smx_context_destroy(_ctx); Smx.Check(rc); }
        }

        GpuTransformerBackend(IntPtr ctx, IntPtr model) { _ctx = ctx; _model = model; }

        // SmqModelLoader.LoadFromSmq(smqPath, config) (SmqModelLoader.cs:29-100): config null
        // takes the GPT-2 configuration from the file's metadata.
        public static GpuTransformerBackend FromSmq(string smqPath, Smx.ModelConfig? config = null, int device = 0)
        {
            Smx.Check(Smx.smx_context_create(device, out IntPtr ctx));
            IntPtr model;
            int rc;
            if (config is Smx.ModelConfig c) rc = Smx.smx_model_load_smq(ctx, smqPath, &c, out model);
            else rc = Smx.smx_model_load_smq(ctx, smqPath, null, out model);
            if (rc != 0) { Smx.smx_context_destroy(ctx); Smx.Check(rc); }
            return new GpuTransformerBackend(ctx, model);
        }

        public GpuSession CreateSession(int maxCtx) => new GpuSession(_model, maxCtx);

        public void Dispose()
        {
            Smx.smx_model_destroy(_model);
            Smx.smx_context_destroy(_ctx);
        }
    }

    // TransformerModel.Forward(idx[1,T], positionOffset) with the KV cache, for one
    // InferenceSession.  Not thread-safe, like the session it serves (SMX_EBUSY otherwise).
    internal sealed unsafe class GpuSession : IDisposable
    {
        readonly IntPtr _s;

        public GpuSession(IntPtr model, int maxCtx) => Smx.Check(Smx.smx_session_create(model, maxCtx, out _s));

        public void ForwardLastRow(ReadOnlySpan<int> tokens, int positionOffset, Span<float> logits)
        {
            fixed (int* t = tokens)
            fixed (float* l = logits)
                Smx.Check(Smx.smx_session_forward(_s, t, tokens.Length, positionOffset, l));
        }

        // Greedy generation on the device.  The prompt is cropped to its last maxCtx tokens by the
        // library (InferenceSession.cs:494-508).  The token's cancellation is forwarded to
        // smx_session_cancel, which the library checks between graph launches; maxTimeMs is
        // ProductionInferenceOptions.MaxTimeMs (0 = none).  A stopped generation throws
        // OperationCanceledException / InferenceTimeoutException like GenerateAsync
        // (InferenceSession.cs:164-172, :287-291); the tokens produced before the stop are in
        // `produced` (the first tokens of the uninterrupted run).
        public int[] GenerateGreedy(ReadOnlySpan<int> prompt, int nNew, CancellationToken cancellationToken = default,
                                    int maxTimeMs = 0)
        {
            return Generate(prompt, nNew, null, 0, cancellationToken, maxTimeMs);
        }

        // As GenerateGreedy, with the reference's sampling pipeline (InferenceSession.cs:565-606).
        public int[] GenerateSampled(ReadOnlySpan<int> prompt, int nNew, in Smx.Sampling options, ulong seed,
                                     CancellationToken cancellationToken = default, int maxTimeMs = 0)
        {
            return Generate(prompt, nNew, options, seed, cancellationToken, maxTimeMs);
        }

        int[] Generate(ReadOnlySpan<int> prompt, int nNew, Smx.Sampling? options, ulong seed,
                       CancellationToken cancellationToken, int maxTimeMs)
        {
            if (maxTimeMs < 0) throw new ArgumentOutOfRangeException(nameof(maxTimeMs));
            cancellationToken.ThrowIfCancellationRequested();
            var outTokens = new int[nNew];
            Smx.GenStats stats = default;
            Smx.Check(Smx.smx_session_set_max_time(_s, maxTimeMs));
            int rc;
            using (cancellationToken.Register(() => Smx.smx_session_cancel(_s)))
            {
                fixed (int* p = prompt)
                fixed (int* o = outTokens)
                {
                    if (options is Smx.Sampling so)
                        rc = Smx.smx_session_generate_sampled(_s, p, prompt.Length, nNew, in so, seed, o, null, &stats);
                    else
                        rc = Smx.smx_session_generate(_s, p, prompt.Length, nNew, o, null, &stats);
                }
            }
            // the registration is disposed: no callback runs from here on.  One that ran after the
            // call had finished left its request pending, which would stop the next call; clear it
            // (smx_session_reset only rewinds the device position, which every call sets itself).
            if (rc == Smx.OK && cancellationToken.IsCancellationRequested) Smx.smx_session_reset(_s);
            if (rc == Smx.ECANCELED || rc == Smx.ETIMEDOUT)
                _produced = outTokens.AsSpan(0, stats.NDecode).ToArray();
            Smx.Check(rc, maxTimeMs);
            _produced = outTokens;
            return outTokens;
        }

        int[] _produced = Array.Empty<int>();
        // The tokens of the last generation, or those produced before it stopped.
        public int[] Produced => _produced;

        public void ResetKVCache() => Smx.Check(Smx.smx_session_reset(_s));

        public void Dispose() => Smx.smx_session_destroy(_s);
    }
}
