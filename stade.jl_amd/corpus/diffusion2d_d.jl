function diffusion2d_d(loss, lossd, u, ud, un, und, n)
    for idx = 1:n * n
        __icse_0 = idx - 1
        i = mod(__icse_0, n) + 1
        j = div(__icse_0, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        __icse_1 = (j - 1) * n
        und[idx] = ud[idx] + 0.1 * ((((ud[__icse_1 + im] + ud[__icse_1 + ip]) + ud[(jm - 1) * n + i]) + ud[(jp - 1) * n + i]) + -(4.0 * ud[idx]))
        un[idx] = u[idx] + 0.1 * (u[__icse_1 + im] + u[__icse_1 + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    for k = 1:n * n
        __cse_2 = un[k]
        lossd[1] = lossd[1] + (2__cse_2) * und[k]
        loss[1] = loss[1] + __cse_2 ^ 2
    end
    return nothing
end

function diffusion2d(loss, u, un, n)
    for idx = 1:n * n
        i = mod(idx - 1, n) + 1
        j = div(idx - 1, n) + 1
        im = mod(i - 2, n) + 1
        ip = mod(i, n) + 1
        jm = mod(j - 2, n) + 1
        jp = mod(j, n) + 1
        un[idx] = u[idx] + 0.1 * (u[(j - 1) * n + im] + u[(j - 1) * n + ip] + u[(jm - 1) * n + i] + u[(jp - 1) * n + i] - 4.0 * u[idx])
    end
    for k = 1:n * n
        loss[1] = loss[1] + un[k] ^ 2
    end
    return nothing
end
